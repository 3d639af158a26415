// NVFP4 GEMV / skinny GEMM for 1..8 activation rows on gfx950 matrix cores.
//
// Semantics: y[m][n] = global * sum_g e4m3(scale[n][g]) * sum_{j in group g} e2m1(code[n][j]) * x[m][j]
// (engine/src/kernels.cpp:48-60 and :116-137; the two CPU branches differ only in FP32 rounding order).
//
// Design (MI355X, bandwidth-bound at M <= 8):
//  - Each wave owns R row-blocks of 16 rows and T k-tiles of 128 inputs; a work-group stacks S waves along k and
//    adds their partials in LDS in a fixed order (deterministic, no atomics). Weights stream as one 16-byte load
//    per lane per tile (a wave reads a contiguous 1 KiB) plus one 2-byte scale load.
//  - Dequantisation is exact and in registers: FP4 -> f16 pairs by v_cvt_scalef32_pk_f16_fp4 (unit scale; the
//    instruction's own scale uses only the exponent), then v_pk_mul_f16 by the E4M3 group scale, which f16 holds
//    exactly; E2M1 x E4M3 products (at most 6 significant bits, 2^-10 .. 2688) are exact in f16.
//  - v_mfma_f32_16x16x32_f16 does the products with FP32 accumulation. The operand's 16 columns carry the high
//    and the low f16 part of up to 8 activation rows (each row first scaled by a power of two), so the FP32
//    activations keep ~22 significant bits at no extra matrix-core cost. Lane (g, c) loads column c's entry
//    4 c + g, so at small m the live columns are a few contiguous lines per MFMA step.
//  - Weights stream with nontemporal loads (read once per call; kept out of the caches' way).
//  - Output: columns 2 r and 2 r + 1 of the accumulator (neighbour lanes) are added, times global and row r's
//    2^-s.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "common.hpp"
#include "kernels.hpp"
#include "nvfp4.hpp"
#include "rowops.hpp"

namespace xtg::hip {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The tile layout from the checkpoint's row-major layout (ModelOpt NVFP4: codes [n][k/2], E4M3 scales [n][k/16]),
// on the device: one wave per tile, lane l takes row rb * 16 + (l & 15), inputs kt * 128 + 32 (l >> 4) .. + 32 (16
// or 32 of them: k is a multiple of 16), zeros for rows past n and inputs past k.
__global__ void __launch_bounds__(256) pack_nvfp4_kernel(const uint8_t* __restrict__ codes,
                                                          const uint8_t* __restrict__ scales, int n, int k, int nb,
                                                          int kt, uint8_t* __restrict__ tiles) {
  const long long tile = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= (long long)nb * kt) return;
  const int l = threadIdx.x & 63, rb = int(tile / kt), t = int(tile % kt);
  const int row = rb * kTileRows + (l & 15), k0 = t * kTileK + 32 * (l >> 4);
  uint2 c0 = make_uint2(0, 0), c1 = make_uint2(0, 0);
  uint32_t s = 0;
  if (row < n && k0 < k) {
    const uint8_t* cr = codes + size_t(row) * size_t(k / 2) + size_t(k0 / 2);   // 8-byte aligned: k / 2 % 8 == 0
    const uint8_t* sr = scales + size_t(row) * size_t(k / 16) + size_t(k0 / 16);
    c0 = *reinterpret_cast<const uint2*>(cr);
    s = sr[0];
    if (k0 + 16 < k) {
      c1 = *reinterpret_cast<const uint2*>(cr + 8);
      s |= uint32_t(sr[1]) << 8;
    }
  }
  uint8_t* dst = tiles + size_t(tile) * kTileBytes;
  *reinterpret_cast<uint4*>(dst + 16 * l) = make_uint4(c0.x, c0.y, c1.x, c1.y);
  *reinterpret_cast<uint16_t*>(dst + 1024 + 2 * l) = uint16_t(s);
}

std::string launch_pack_nvfp4(const uint8_t* codes, const uint8_t* scales, int n, int k, uint8_t* tiles,
                              hipStream_t stream) {
  const int nb = (n + kTileRows - 1) / kTileRows, kt = (k + kTileK - 1) / kTileK;
  const long long waves = (long long)nb * kt;
  hipLaunchKernelGGL(pack_nvfp4_kernel, dim3(unsigned((waves + 3) / 4)), dim3(256), 0, stream, codes, scales, n, k,
                     nb, kt, tiles);
  HIP_CHECK(hipGetLastError());
  return "pack_nvfp4_kernel";
}

// ---------------------------------------------------------------------------------------- activation operand

__device__ inline float load_x(const void* x, int x_dtype, size_t i) {
  if (x_dtype == kXBF16) {
    const uint32_t b = uint32_t(static_cast<const uint16_t*>(x)[i]) << 16;
    return __uint_as_float(b);
  }
  return static_cast<const float*>(x)[i];
}

// Eight consecutive inputs of row j from chunk c (inputs 8c .. 8c + 7); zeros past k (k is a multiple of 16, so
// a chunk is either whole or past the end).
__device__ inline void load_chunk(const void* x, int x_dtype, int j, int k, int c, float v[8]) {
  const int k0 = c * 8;
  if (k0 >= k) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
    return;
  }
  const size_t base = size_t(j) * size_t(k) + size_t(k0);
  if (x_dtype == kXBF16) {
    const uint4 b = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base);
    const uint32_t w[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + base);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + base + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
}

// One work-group per activation row: the row's largest magnitude picks the power of two 2^e that brings it to
// [2^14, 2^15); the scaled row is split into f16 high and low parts in MFMA B-operand order (columns 2 jj and
// 2 jj + 1 of its group of 8 rows: row j is row jj = j % 8 of group j / 8, whose operand starts at
// op + (j / 8) * op_group_bytes(k)). Rows up to 8192 wide make one read of x (chunks held in registers); wider
// rows read x twice. Columns of rows >= m are not written: the GEMV and the GEMM never use them. copy (FP32 rows
// only, or NULL): the rows are also written there as they are read.
constexpr int kPrepThreads = 256, kPrepChunks = 4;
__global__ void __launch_bounds__(kPrepThreads) prep_x_kernel(const void* __restrict__ x, int x_dtype, int k, int kt,
                                                              char* __restrict__ op, size_t stride,
                                                              float* __restrict__ copy) {
  __shared__ float red[kPrepThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  f16x8* __restrict__ xop = reinterpret_cast<f16x8*>(op + size_t(row / kMaxRows) * stride);
  float* __restrict__ xinv = reinterpret_cast<float*>(op + size_t(row / kMaxRows) * stride + size_t(kt) * 4096);
  const int j = row % kMaxRows;
  const int chunks = kt * 16;
  float v[kPrepChunks][8];
  float mx = 0.f;
#pragma unroll
  for (int u = 0; u < kPrepChunks; ++u) {
    const int c = tid + u * kPrepThreads;
    load_chunk(x, x_dtype, row, k, c < chunks ? c : chunks, v[u]);
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[u][i]));
  }
  if (copy) {
#pragma unroll
    for (int u = 0; u < kPrepChunks; ++u) {
      const int c = tid + u * kPrepThreads;
      if (c * 8 < k) {
        float* d = copy + size_t(row) * size_t(k) + size_t(c) * 8;
        *reinterpret_cast<float4*>(d) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
        *reinterpret_cast<float4*>(d + 4) = make_float4(v[u][4], v[u][5], v[u][6], v[u][7]);
      }
    }
  }
  for (int c = tid + kPrepChunks * kPrepThreads; c < chunks; c += kPrepThreads) {
    float w[8];
    load_chunk(x, x_dtype, row, k, c, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(w[i]));
    if (copy && c * 8 < k) {
      float* d = copy + size_t(row) * size_t(k) + size_t(c) * 8;
      *reinterpret_cast<float4*>(d) = make_float4(w[0], w[1], w[2], w[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(w[4], w[5], w[6], w[7]);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < kPrepThreads / 64; ++i) mx = fmaxf(mx, red[i]);
  const int e = operand_exponent(mx);
  const float up = ldexpf(1.f, e);
  if (tid == 0) xinv[j] = ldexpf(1.f, -e);
#pragma unroll
  for (int u = 0; u < kPrepChunks; ++u) {
    const int c = tid + u * kPrepThreads;
    if (c < chunks) store_chunk(xop, j, c, v[u], up);
  }
  for (int c = tid + kPrepChunks * kPrepThreads; c < chunks; c += kPrepThreads) {
    float w[8];
    load_chunk(x, x_dtype, row, k, c, w);
    store_chunk(xop, j, c, w, up);
  }
}

std::string launch_prep_x(const void* x, int x_dtype, int m, int k, void* op, hipStream_t stream, float* copy) {
  XTG_CHECK(m >= 1, "prep_x: %d rows", m);
  XTG_CHECK(k > 0 && k % 16 == 0, "prep_x: width %d (a multiple of 16)", k);
  XTG_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, "prep_x: activations at %p are not 16-byte aligned", x);
  XTG_CHECK(!copy || (x_dtype == kXF32 && reinterpret_cast<uintptr_t>(copy) % 16 == 0),
            "prep_x: a copy is of FP32 rows, 16-byte aligned");
  const int kt = (k + kTileK - 1) / kTileK;
  hipLaunchKernelGGL(prep_x_kernel, dim3(unsigned(m)), dim3(kPrepThreads), 0, stream, x, x_dtype, k, kt,
                     static_cast<char*>(op), op_group_bytes(k), copy);
  HIP_CHECK(hipGetLastError());
  return "prep_x_kernel";
}

// ------------------------------------------------------------------------------------------------------ GEMV

struct GemvArgs {
  // what a work-group needs before its first load, in the first two 64-byte lines: the work-group -> weight choice
  // reads wg_end and then nb / tiles from the same line
  int wg_end[4];   // cumulative work-group counts per weight
  int nb[4];
  const uint8_t* tiles[4];
  int nw;
  int kt;
  int m;
  int k;
  int waves;           // waves per work-group (blockDim.x / 64)
  const void* x;       // raw rows [m][k] (FP32 or BF16) when the kernel builds its own operand
  const uint4* xop;
  const float* xinv;   // the operand's row factors (NULL: the rows were taken raw)
  float* y;
  long long y_part;    // with a K split in two: the floats from one output set to the next (blockIdx.y)
  // the epilogue's
  int n[4];
  float global[4];
  long long y_off[4];
  const float* col_scale[4];   // optional per-output-column factor (the LM head's logit scale)
#ifdef XTG_PHASE_STAMPS
  unsigned long long* stamps;   // per-wave phase records (the phase-stamp build only)
  long long stamp_records;
#endif
};

// Phase stamps (the phase-stamp build only, build.py --stamps, -DXTG_PHASE_STAMPS): each wave of gemv_kernel reads
// the constant-rate clock (s_memrealtime) at kernel entry [0], once its loads are issued [1], when its first row
// load has arrived [7] (raw rows), once its operand is built [2], when its first weight tile has arrived [3], after
// its matrix ops [4], after the work-group's barrier [5] and after its stores are issued [6]; lane 0 writes the 8
// stamps as one record at ((blockIdx.y * gridDim.x + blockIdx.x) * 16 + wave). A stamp that waits on a value (an empty asm statement taking
// it) marks when that value is there; the loads themselves are issued as in the product build.
#ifdef XTG_PHASE_STAMPS
#define XTG_STAMPS_DECL unsigned long long st_[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#define XTG_STAMP(i) st_[i] = __builtin_amdgcn_s_memrealtime();
#define XTG_STAMP_AFTER(i, v)        \
  {                                  \
    asm volatile("" ::"v"(v));       \
    st_[i] = __builtin_amdgcn_s_memrealtime(); \
  }
#define XTG_STAMPS_WRITE                                                                                        \
  {                                                                                                             \
    st_[6] = __builtin_amdgcn_s_memrealtime();                                                                  \
    const long long rec_ = ((long long)blockIdx.y * gridDim.x + blockIdx.x) * 16 + wave;                        \
    if (a.stamps && lane == 0 && rec_ < a.stamp_records) {                                                      \
      unsigned long long* d_ = a.stamps + rec_ * 8;                                                             \
      for (int i_ = 0; i_ < 8; ++i_) d_[i_] = st_[i_];                                                          \
    }                                                                                                           \
  }
namespace {
unsigned long long* g_stamp_buf = nullptr;   // set by xtg_hip_phase_stamps (host side)
long long g_stamp_records = 0;
}  // namespace
#else
#define XTG_STAMPS_DECL
#define XTG_STAMP(i)
#define XTG_STAMP_AFTER(i, v)
#define XTG_STAMPS_WRITE
#endif

// Output of one accumulator fragment: for activation row j, rows 4 g .. 4 g + 3 of the row-block (high and low
// columns already added).
__device__ inline void store_rows(const GemvArgs& a, int wi, int rb, int g, int j, f32x4 v) {
  if (j >= a.m) return;
  const int n = a.n[wi];
  const int n0 = rb * kTileRows + 4 * g;
  const float f = a.xinv ? a.global[wi] * a.xinv[j] : a.global[wi];
  float* yp = a.y + a.y_off[wi] + (long long)blockIdx.y * a.y_part + (long long)j * n;
  const float* cs = a.col_scale[wi];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (n0 + e < n) yp[n0 + e] = cs ? (v[e] * f) * cs[n0 + e] : v[e] * f;
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Lanes of one wave passing values through LDS: a wave's LDS operations execute in issue order, so keeping the
// compiler's order is enough.
__device__ inline void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The operand of a wave's T k-tiles from raw BF16 rows, converted by all 64 lanes and staged through LDS one k-tile
// at a time. Lane (j, i) = (lane / 16, lane % 16) holds inputs 8 i .. 8 i + 7 of each k-tile of row j in xr[u][0]
// and of row j + 4 in xr[u][1] (zeros for rows past m). Each row's inputs are scaled by the power of two 2^e that
// brings the row's largest magnitude over the wave's k-tiles to [2^14, 2^15) (prep_x_kernel's rule, per wave's
// share of the row instead of per row; the row's 16 lanes agree on it through DPP within their row of lanes), so
// the matrix ops accumulate across the wave's k-tiles and one multiply by 2^-e per column follows. BF16 carries 8
// significant bits, so f16(x * 2^e) is exact wherever it is a normal f16 and the low part is zero (the odd operand
// columns read zeros). An input whose scaled value falls below f16's normal range (at least 2^28 times smaller than
// that largest magnitude) is flushed, an error below 2^-28 of it; e is capped at 112 so the exponent shift stays a
// subtraction (rows whose largest magnitude is under 2^-98 keep at least 6 of f16's 11 bits above their largest
// value, still more than BF16's 8). With the abs bits a = [E:8][M:7], the f16 of x * 2^e is [E - 112 + e : 5][M : 7]
// [000]: a saturating subtraction of (112 - e) << 7 (0 when the result would be below the normal range), a shift by 3
// and the sign put back. A row holding an infinity or NaN gets the factor NaN (NaN outputs, as the prepared operand
// gives). Each staged k-tile [8 rows][16][8 f16] then goes to the lanes that consume it: lane (c, g) of the matrix
// op's operand takes row c / 2's inputs 32 g .. 32 g + 31 (four steps of 8) for even c < 2 m, zeros else. One
// exponent per wave instead of per k-tile halves the conversion's instructions (the largest magnitude is reduced
// across lanes once): the 8-row calls of the 4B layer's projections took 0.14-0.65 us less per launch.
constexpr int kStageVecs = 8 * 16 + 2;   // one wave's staging, in 16-byte units: the rows' k-tile, then 8 factors

__device__ inline uint32_t row16_max(uint32_t v) {
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppXor1, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppXor2, 0xF, 0xF, false)));
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppHalfMirror, 0xF, 0xF, false)));
  return max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), kDppMirror, 0xF, 0xF, false)));
}

// The operand entries xb[u][step] of lane (col, grp) for the wave's T k-tiles and the lane's column factor 2^-e (1
// for dead columns), from the rows in xr (lane layout above); stage: this wave's kStageVecs, free on entry and again
// on return.
template <int T>
__device__ inline float bf16_operands(uint4 (&xr)[T][2], int m, int lane, uint4* stage, uint4 (&xb)[T][4]) {
  const int j = lane >> 4, i = lane & 15, col = lane & 15, grp = lane >> 4;
  float* fac = reinterpret_cast<float*>(stage + 128);
  u16x2 c2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {   // rows j and j + 4: the largest magnitude over the wave's k-tiles
    u16x2 m2 = {0, 0};
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const uint32_t w[4] = {xr[u][h].x, xr[u][h].y, xr[u][h].z, xr[u][h].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, w[q] & 0x7fff7fffu));
    }
    const uint32_t mx = row16_max(m2.x > m2.y ? uint32_t(m2.x) : uint32_t(m2.y));
    const int e = mx == 0 || mx >= 0x7f80u ? 0 : min(141 - int(mx >> 7), 112);
    const unsigned short c = (unsigned short)((112 - e) << 7);
    c2[h] = u16x2{c, c};
    if (i == 0 && (h == 0 || m > 4)) fac[j + 4 * h] = mx >= 0x7f80u ? __builtin_nanf("") : ldexpf(1.f, -e);
  }
  const int r = col >> 1;
  const bool live = (col & 1) == 0 && r < m;
  const int rc = live ? r : 0;
  float xs = 1.f;
#pragma unroll
  for (int u = 0; u < T; ++u) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && m <= 4) break;   // uniform: the second half of the rows
      uint32_t w[4] = {xr[u][h].x, xr[u][h].y, xr[u][h].z, xr[u][h].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u16x2 d = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, w[q] & 0x7fff7fffu), c2[h]);
        const u16x2 f = d << (unsigned short)3;
        w[q] = (w[q] & 0x80008000u) | __builtin_bit_cast(uint32_t, f);
      }
      stage[(j + 4 * h) * 16 + i] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    wave_lds_order();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 v = stage[rc * 16 + 4 * grp + t];
      xb[u][t] = live ? v : make_uint4(0, 0, 0, 0);
    }
    if (u == 0) xs = live ? fac[rc] : 1.f;
    wave_lds_order();   // read before the next k-tile's staging
  }
  return xs;
}

// XR: false = a prepared operand (xop / xinv); true = raw BF16 rows (the kernel builds the operand per k-tile in
// registers, so no separate prep pass runs). FP32 rows keep the prepared operand: their high / low split costs
// more per wave than the separate prep launch saves.
template <int R, int T, int MAXT, bool XR>
__global__ void __launch_bounds__(MAXT) gemv_kernel(const GemvArgs a) {
  extern __shared__ f32x4 red[];
  XTG_STAMPS_DECL
  XTG_STAMP(0)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, S = a.waves;
  int wi = 0;
  while (wi < 3 && int(blockIdx.x) >= a.wg_end[wi]) ++wi;   // wg_end past the last weight = the total
  const int rb0 = (int(blockIdx.x) - (wi ? a.wg_end[wi - 1] : 0)) * R;
  const int nb = a.nb[wi], KT = a.kt;
  const uint8_t* __restrict__ tiles = a.tiles[wi];
  const int kt0 = (int(blockIdx.y) * S + wave) * T;   // with a K split, blockIdx.y's half of the k-tiles

  // every load of the wave first (T k-tiles of activations, R x T weight tiles), then the math; operand columns
  // of absent activation rows are not loaded (their accumulator columns are never stored)
  const int col = lane & 15, grp = lane >> 4;
  const bool live_col = (col >> 1) < a.m;
  const int entry = 4 * col + grp;
  uint4 xb[T][4];
  uint4 cw[T][R];
  uint32_t sw[T][R];
  // raw rows: lane (j, i) = (lane / 16, lane % 16) loads inputs 8 i .. 8 i + 7 of each k-tile of rows j and j + 4
  // (8 BF16 per load; k is a multiple of 16, so a load is wholly inside the row or wholly past its end)
  uint4 xr[XR ? T : 1][2];
  if constexpr (XR) {
    // the raw rows first, so they are turned into the operand while the weights are in flight; buffer loads
    // return zeros past the rows (absent rows, k-tiles past k), so no load sits behind a branch
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(a.x), (short)0, a.m * a.k * 2, 0x00020000);
    const int j = lane >> 4, i = lane & 15;
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const int kt = kt0 + u;
      const int ki = kt * kTileK + 8 * i;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = j + 4 * h;
        const bool in = kt < KT && row < a.m && ki < a.k;
        const uint32_t off = in ? (uint32_t(row) * uint32_t(a.k) + uint32_t(ki)) * 2u : 0x80000000u;
        xr[u][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, int(off), 0, 0));
      }
    }
  }
#pragma unroll
  for (int u = 0; u < T; ++u) {
    const int kt = kt0 + u;
    const bool ok = kt < KT;
    if constexpr (!XR) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        xb[u][t] = ok && live_col ? a.xop[(size_t(kt) * 4 + size_t(t)) * 64 + size_t(entry)] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool ok2 = ok && rb0 + r < nb;
      if constexpr (XR) {
        // branch-free, so the conversion can wait for the rows alone: an absent tile loads a tile of the same
        // weight (clamped) and is used as it is: past the last row-block its results are not stored, past k its
        // products meet zero inputs
        (void)ok2;
        const uint8_t* tile =
            tiles + (size_t(min(rb0 + r, nb - 1)) * size_t(KT) + size_t(min(kt, KT - 1))) * kTileBytes;
        const u32x4 c4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + 16 * lane));
        cw[u][r] = make_uint4(c4[0], c4[1], c4[2], c4[3]);
        sw[u][r] = uint32_t(__builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(tile + 1024 + 2 * lane)));
        continue;
      }
      const uint8_t* tile = tiles + (size_t(rb0 + r) * size_t(KT) + size_t(kt)) * kTileBytes;
      if (ok2) {
        const u32x4 c4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + 16 * lane));
        cw[u][r] = make_uint4(c4[0], c4[1], c4[2], c4[3]);
        sw[u][r] = uint32_t(__builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(tile + 1024 + 2 * lane)));
      } else {
        cw[u][r] = make_uint4(0, 0, 0, 0);
        sw[u][r] = 0u;
      }
    }
  }
  float xs = 1.f;   // raw rows: the wave's factor 2^-e for the lane's column
#ifdef XTG_PHASE_STAMPS
  __builtin_amdgcn_sched_barrier(0);
  XTG_STAMP(1)
#endif
  if constexpr (XR) {
    XTG_STAMP_AFTER(7, xr[0][0].x)
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the conversion waits on x
    // this wave's staging area, after the cross-wave sums' region
    uint4* stage = reinterpret_cast<uint4*>(red) + (S > 1 ? S * R * kMaxRows * 4 : 0) + wave * kStageVecs;
    xs = bf16_operands<T>(xr, a.m, lane, stage, xb);
  }
  if constexpr (XR) {
    XTG_STAMP_AFTER(2, xb[T - 1][3].x)
  }
  XTG_STAMP_AFTER(3, cw[0][0].x)
  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < T; ++u) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f16x2 s0 = scale_pair(sw[u][r], 0), s1 = scale_pair(sw[u][r], 1);
      const uint32_t words[4] = {cw[u][r].x, cw[u][r].y, cw[u][r].z, cw[u][r].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f16x8 A = dequant8(words[t], t < 2 ? s0 : s1);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(f16x8, xb[u][t]), acc[r], 0, 0, 0);
      }
    }
  }
  if constexpr (XR)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] *= xs;   // a power of two: exact
  XTG_STAMP_AFTER(4, acc[R - 1][3])
  if (S == 1) {
    XTG_STAMP(5)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f32x4 v = acc[r];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += dpp<kDppXor1>(v[e]);   // high + low column of the row
      if ((col & 1) == 0 && rb0 + r < nb) store_rows(a, wi, rb0 + r, grp, col >> 1, v);
    }
    XTG_STAMPS_WRITE
    return;
  }
  // each wave adds its high and low columns (lanes l and l ^ 1) and stores row j's sums at [wave][r][j][gg]
#pragma unroll
  for (int r = 0; r < R; ++r) {
    f32x4 v = acc[r];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += dpp<kDppXor1>(v[e]);
    if ((col & 1) == 0 && (col >> 1) < a.m) red[((wave * R + r) * kMaxRows + (col >> 1)) * 4 + grp] = v;
  }
  __syncthreads();
  XTG_STAMP(5)
  for (int item = threadIdx.x; item < R * 32; item += S * 64) {
    const int r = item >> 5, l = item & 31, gg = l >> 3, jj = l & 7;
    if (rb0 + r >= nb || jj >= a.m) continue;
    // the S <= 16 waves in order, the reads in batches of 4 with clamped indices (no wait between them)
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w0 = 0; w0 < 16; w0 += 4) {
      if (w0 >= S) break;
      f32x4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = red[(((w0 + i < S ? w0 + i : S - 1) * R + r) * kMaxRows + jj) * 4 + gg];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (w0 + i < S) sum += v[i];
    }
    store_rows(a, wi, rb0 + r, gg, jj, sum);
  }
  XTG_STAMPS_WRITE
}

// ------------------------------------------------------------- one or two BF16 rows on the block-scaled FP4 op
//
// gfx950's v_mfma_scale_f32_16x16x128_f8f6f4 multiplies E2M1 codes as they are stored (A: 16 weight rows x 128
// inputs, lane l = row l % 16 holding inputs 32 (l / 16) .. + 31 as 16 bytes, low nibble first: exactly a lane's
// share of a weight tile) with an FP8 E4M3 operand B whose lanes (column l % 16, q = l / 16) hold inputs 16 q .. + 15
// in bytes 0..15 and 64 + 16 q .. + 15 in bytes 16..31, each column scaled by a power of two (E8M0). So no
// dequantisation runs on the vector ALUs. The NVFP4 group scale (E4M3, per 16 inputs) is not a power of two, so
// the group sums are kept apart: column c of the operand holds activation row j's group g = c % 8 of the k-tile
// (zeros elsewhere) as part p = c / 8 -- a BF16 input x (8 significant bits) is hi + lo / 16 exactly, hi = E4M3 of
// x 2^e (the group's largest magnitude brought to [2^7, 2^8)) and lo = E4M3 of (x 2^e - hi) 16, the remainder
// having at most 4 significant bits -- with column scale 2^-e (hi) or 2^-(e + 4) (lo). Output (row n, column c)
// is then the exact-product FP32 sum over one group and part; each lane multiplies its four rows by their E4M3
// group scale and accumulates over the k-tiles, and the 16 columns are added by DPP at the end.
// Inputs whose scaled magnitude falls below E4M3's subnormal range (2^-20 of the group's largest) lose bits below
// 2^-13 of that scale. A group holding an infinity or NaN gets NaN codes (NaN outputs).
// Lane layout of the staging: lane l converts inputs 2 l, 2 l + 1 of each row (one 32-bit load), its group being
// the 8 lanes l / 8 (largest magnitude by DPP within the half-row), and writes the two planes (hi, lo) [MR][128]
// bytes and the groups' exponents to LDS; lane (c, q) then reads group c % 8 of plane c / 8 (16 bytes).
constexpr int kMxStageVecs = (2 * 2 * 128 + 2 * 8 * 4) / 16;   // two rows: [2 planes][2 rows][128 B] + [2][8] ints

template <int R, int T, int MAXT, int MR>
__global__ void __launch_bounds__(MAXT) gemv_mx_kernel(const GemvArgs a) {
  extern __shared__ f32x4 red[];
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, S = a.waves;
  int wi = 0;
  while (wi < 3 && int(blockIdx.x) >= a.wg_end[wi]) ++wi;   // wg_end past the last weight = the total
  const int rb0 = (int(blockIdx.x) - (wi ? a.wg_end[wi - 1] : 0)) * R;
  const int nb = a.nb[wi], KT = a.kt;
  const uint8_t* __restrict__ tiles = a.tiles[wi];
  const int kt0 = wave * T;
  const int col = lane & 15, q = lane >> 4, g = col & 7, p = col >> 3;

  // every load first: each row's two inputs of every k-tile (zeros for absent rows and k-tiles past k), then the
  // weight tiles (clamped: an absent tile is a tile of the same weight, its results unstored or met by zeros) with
  // the 8 scale bytes this lane's output rows need (rows 4 q .. 4 q + 3, group g)
  uint32_t xr[T][MR];
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.x), (short)0, a.m * a.k * 2, 0x00020000);
#pragma unroll
  for (int u = 0; u < T; ++u) {
    const int ki = (kt0 + u) * kTileK + 2 * lane;
#pragma unroll
    for (int j = 0; j < MR; ++j) {
      const bool in = kt0 + u < KT && j < a.m && ki < a.k;
      const uint32_t off = in ? (uint32_t(j) * uint32_t(a.k) + uint32_t(ki)) * 2u : 0x80000000u;
      xr[u][j] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(xres, int(off), 0, 0));
    }
  }
  u32x4 cw[T][R];
  u32x2 sw[T][R];
#pragma unroll
  for (int u = 0; u < T; ++u) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* tile =
          tiles + (size_t(min(rb0 + r, nb - 1)) * size_t(KT) + size_t(min(kt0 + u, KT - 1))) * kTileBytes;
      cw[u][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + 16 * lane));
      sw[u][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(tile + 1024 + 32 * (g >> 1) + 8 * q));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  uint8_t* stage = reinterpret_cast<uint8_t*>(reinterpret_cast<uint4*>(red) + (S > 1 ? S * R * kMaxRows * 4 : 0) +
                                              wave * kMxStageVecs);
  int* gexp = reinterpret_cast<int*>(stage + 2 * MR * 128);
  f32x4 acc[R][MR];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < MR; ++j) acc[r][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < T; ++u) {
    i32x8 B[MR];
    int sb[MR];
#pragma unroll
    for (int j = 0; j < MR; ++j) {
      const uint32_t w = xr[u][j];
      uint32_t am = max(w & 0x7fffu, (w >> 16) & 0x7fffu);
      am = max(am, uint32_t(__builtin_amdgcn_update_dpp(0, int(am), kDppXor1, 0xF, 0xF, false)));
      am = max(am, uint32_t(__builtin_amdgcn_update_dpp(0, int(am), kDppXor2, 0xF, 0xF, false)));
      am = max(am, uint32_t(__builtin_amdgcn_update_dpp(0, int(am), kDppHalfMirror, 0xF, 0xF, false)));
      const bool fin = am < 0x7f80u;
      const int e = am == 0u || !fin ? 0 : min(134 - int(am >> 7), 123);
      const float v0 = ldexpf(__uint_as_float(w << 16), e), v1 = ldexpf(__uint_as_float(w & 0xffff0000u), e);
      uint32_t hi = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false)) & 0xffffu;
      const float l0 = (v0 - __builtin_amdgcn_cvt_f32_fp8(hi, 0)) * 16.f;
      const float l1 = (v1 - __builtin_amdgcn_cvt_f32_fp8(hi, 1)) * 16.f;
      uint32_t lo = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(l0, l1, 0, false)) & 0xffffu;
      if (!fin) hi = 0x7f7fu, lo = 0u;
      *reinterpret_cast<uint16_t*>(stage + j * 128 + 2 * lane) = uint16_t(hi);
      *reinterpret_cast<uint16_t*>(stage + (MR + j) * 128 + 2 * lane) = uint16_t(lo);
      if ((lane & 7) == 0) gexp[j * 8 + (lane >> 3)] = e;
    }
    wave_lds_order();
#pragma unroll
    for (int j = 0; j < MR; ++j) {
      const uint4 b = *reinterpret_cast<const uint4*>(stage + (p * MR + j) * 128 + 16 * g);
      const bool first = g == q, second = g == q + 4;
      B[j] = i32x8{int(first ? b.x : 0u), int(first ? b.y : 0u), int(first ? b.z : 0u), int(first ? b.w : 0u),
                   int(second ? b.x : 0u), int(second ? b.y : 0u), int(second ? b.z : 0u), int(second ? b.w : 0u)};
      sb[j] = 127 - gexp[j * 8 + g] - 4 * p;
    }
    wave_lds_order();   // read before the next k-tile's staging
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const i32x8 A = {int(cw[u][r][0]), int(cw[u][r][1]), int(cw[u][r][2]), int(cw[u][r][3]), 0, 0, 0, 0};
      const uint32_t s0 = sw[u][r][0] >> (8 * (g & 1)), s1 = sw[u][r][1] >> (8 * (g & 1));
      const f32x4 s = f32x4{__builtin_amdgcn_cvt_f32_fp8(s0, 0), __builtin_amdgcn_cvt_f32_fp8(s0, 2),
                            __builtin_amdgcn_cvt_f32_fp8(s1, 0), __builtin_amdgcn_cvt_f32_fp8(s1, 2)};
#pragma unroll
      for (int j = 0; j < MR; ++j) {
        const f32x4 c = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B[j], f32x4{0.f, 0.f, 0.f, 0.f}, 4, 0,
                                                                          0, 127, 0, sb[j]);
        acc[r][j] += c * s;
      }
    }
  }
  // the 16 columns (8 groups x hi / lo) of each output row added within each row of lanes; lane (c, q) with c = 2 j
  // then holds activation row j's sums for output rows 4 q .. 4 q + 3, the layout of gemv_kernel's epilogue
  f32x4 v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int j = 0; j < MR; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = acc[r][j][e];
        t += dpp<kDppXor1>(t);
        t += dpp<kDppXor2>(t);
        t += dpp<kDppHalfMirror>(t);
        t += dpp<kDppMirror>(t);
        acc[r][j][e] = t;
      }
    }
    v[r] = acc[r][0];
    if constexpr (MR > 1) v[r] = col >= 2 ? acc[r][1] : acc[r][0];
  }
  const bool store_lane = (col & 1) == 0 && (col >> 1) < min(a.m, MR);
  if (S == 1) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (store_lane && rb0 + r < nb) store_rows(a, wi, rb0 + r, q, col >> 1, v[r]);
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (store_lane) red[((wave * R + r) * kMaxRows + (col >> 1)) * 4 + q] = v[r];
  __syncthreads();
  for (int item = threadIdx.x; item < R * 32; item += S * 64) {
    const int r = item >> 5, l = item & 31, gg = l >> 3, jj = l & 7;
    if (rb0 + r >= nb || jj >= min(a.m, MR)) continue;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w0 = 0; w0 < 16; w0 += 4) {
      if (w0 >= S) break;
      f32x4 t[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = red[(((w0 + i < S ? w0 + i : S - 1) * R + r) * kMaxRows + jj) * 4 + gg];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (w0 + i < S) sum += t[i];
    }
    store_rows(a, wi, rb0 + r, gg, jj, sum);
  }
}

namespace {
using GemvFn = void (*)(const GemvArgs);

// Raw BF16 rows hold 16 inputs (8 VGPRs) per lane and k-tile until the tile's operand is built. Kernels that would
// exceed a 1024-thread group's 128 VGPRs or take more than 4 k-tiles per wave are not made (those calls take the
// prepared operand), nor two row-blocks of four k-tiles in 1024-thread groups (measured slower than one).
template <int R, int T>
GemvFn pick_fn(int threads, bool xr) {
  if (xr) {
    if constexpr (T <= 4) {
      if (threads <= 512) return gemv_kernel<R, T, 512, true>;
      if constexpr (T <= 2 || R == 1) return gemv_kernel<R, T, 1024, true>;
    }
    return nullptr;
  }
  if (threads <= 512) return gemv_kernel<R, T, 512, false>;
  return gemv_kernel<R, T, 1024, false>;
}

GemvFn gemv_fn(int r, int t, int threads, bool xr = false) {
#define XTG_CASE(R, T) \
  if (r == R && t == T) return pick_fn<R, T>(threads, xr);
  XTG_CASE(1, 1) XTG_CASE(1, 2) XTG_CASE(1, 3) XTG_CASE(1, 4) XTG_CASE(1, 6) XTG_CASE(1, 8)
  XTG_CASE(2, 1) XTG_CASE(2, 2) XTG_CASE(2, 3) XTG_CASE(2, 4) XTG_CASE(2, 6)
  XTG_CASE(4, 1) XTG_CASE(4, 2) XTG_CASE(4, 3)
#undef XTG_CASE
  return nullptr;
}

bool shape_ok(int r, int t, int s, bool raw = false) {
  if (s < 1 || s > 16) return false;
  if (r * t > 12) return false;
  if (s > 8 && t > 4) return false;   // 1024-thread groups get 128 VGPRs per lane: T > 4 spills there
  return gemv_fn(r, t, s * 64, raw) != nullptr;
}

template <int R, int T, int MR>
GemvFn mx_pick(int threads) {
  if (threads <= 512) return gemv_mx_kernel<R, T, 512, MR>;
  return gemv_mx_kernel<R, T, 1024, MR>;
}

// the block-scaled FP4 kernel for one or two raw BF16 rows, at the shapes the raw-row kernel takes
GemvFn gemv_mx_fn(int r, int t, int threads, int m) {
#define XTG_CASE(R, T)                                             \
  if (r == R && t == T) return m == 1 ? mx_pick<R, T, 1>(threads) : mx_pick<R, T, 2>(threads);
  XTG_CASE(1, 2) XTG_CASE(1, 4) XTG_CASE(2, 2) XTG_CASE(2, 4) XTG_CASE(4, 2) XTG_CASE(4, 4)
#undef XTG_CASE
  return nullptr;
}

// XTG_GEMV_MX=0 keeps one and two BF16 rows on the f16 matrix op (for comparison)
bool mx_enabled() {
  static const bool on = [] {
    const char* env = std::getenv("XTG_GEMV_MX");
    return !(env && env[0] == '0');
  }();
  return on;
}
}  // namespace

GemvShape gemv_shape(int kt, const int* nbs, int nw, int m, bool raw) {
  if (const char* env = std::getenv("XTG_GEMV_SHAPE")) {   // "R,T": a fixed shape for experiments
    int r = 0, t = 0;
    if (std::sscanf(env, "%d,%d", &r, &t) == 2) {
      const int s = (kt + t - 1) / t;
      if (shape_ok(r, t, s, raw)) return {r, t, s};
    }
  }
  if (raw) {
    // raw BF16 rows (measured the same way, rotated cold weights, launch-shape sweeps over the decode projections
    // at M = 1, 2, 4, 8): four row-blocks per wave with many row-blocks, two with few, and four k-tiles per wave
    // (with one row-block) only where K needs them (16 waves at most per work-group)
    int nb = 0;
    for (int i = 0; i < nw; ++i) nb += nbs[i];
    // (one row-block per wave where the launch fits one work-group per CU: 3072 x 3072 at M = 4 / 8, 4.96 / 5.46
    // -> 4.42 / 4.74 us)
    int r = nb <= 256 ? 1 : nb >= 512 ? 4 : 2;
    const int t = (kt + 1) / 2 <= 16 ? 2 : 4;
    // one or two rows on the block-scaled op (measured the same way over configs 0 and 1): one row-block per wave
    // while the launch fits one work-group per CU, four where two would leave the CUs unevenly loaded (512 < nb <
    // 1024), two otherwise (two work-groups per CU at 1024)
    if (m <= 2 && mx_enabled()) r = nb <= 256 ? 1 : (nb <= 512 || nb >= 1024) ? 2 : 4;
    if (shape_ok(r, t, (kt + t - 1) / t, true)) return {r, t, (kt + t - 1) / t};
    if (shape_ok(1, 4, (kt + 3) / 4, true)) return {1, 4, (kt + 3) / 4};
  }
  // The k-split -- T k-tiles per wave, S = ceil(kt / T) waves added in a fixed order -- fixes every output's
  // summation order, so it depends on k alone: a weight's outputs are bit-identical alone and fused with others
  // (the reference's device test, tests/opencl_test.cpp:24-31). Two k-tiles per wave up to 32, four up to 64,
  // then six or eight (those spill in 1024-thread groups: slower, still exact). The row-blocks per wave only
  // choose which rows a wave computes: measured on MI355X (rotated cold weights, launch-shape sweeps over the
  // decode projections), many row-blocks want two per wave (four at M >= 4, where the activation operand is
  // wider and reused across more rows), few want one.
  int nb = 0, nb_min = nbs[0];
  for (int i = 0; i < nw; ++i) nb += nbs[i], nb_min = std::min(nb_min, nbs[i]);
  // very tall weights only (LM heads), each of them: the most bytes in flight per wave that still fits 512-thread
  // groups, four row-blocks x three k-tiles (64% of HBM peak on 131072 x 3072 at M=1, against 59% for 2 x 2)
  if (nb_min >= 4096 && kt <= 24 && shape_ok(4, 3, (kt + 2) / 3)) return {4, 3, (kt + 2) / 3};
  int t = 0;
  for (int tt : {2, 4, 6, 8})
    if (!t && (kt + tt - 1) / tt <= 16 && gemv_fn(1, tt, 1024) != nullptr) t = tt;
  XTG_CHECK(t != 0, "gemv: %d k-tiles (K up to 16384)", kt);
  const int s = (kt + t - 1) / t;
  int r = nb >= 512 ? (m >= 4 ? 4 : 2) : 1;
  while (r > 1 && !shape_ok(r, t, s)) r /= 2;
  return {r, t, s};
}

namespace {
bool raw_kind(const GemvCall& c) { return c.x && c.x_dtype == kXBF16; }

GemvShape call_shape(const GemvCall& c) {
  int nbs[4];
  for (int i = 0; i < c.nw; ++i) nbs[i] = c.w[i]->nb;
  return gemv_shape(c.w[0]->kt, nbs, c.nw, c.m, raw_kind(c));
}
}  // namespace

bool gemv_takes_raw(const GemvCall& c) {
  if (!raw_kind(c) || c.m < 1 || c.m > kMaxRows || reinterpret_cast<uintptr_t>(c.x) % 16 != 0) return false;
  const GemvShape sh = call_shape(c);
  return gemv_fn(sh.r, sh.t, sh.s * 64, raw_kind(c)) != nullptr;
}

std::string launch_gemv(const GemvCall& c, hipStream_t stream) {
  XTG_CHECK(c.nw >= 1 && c.nw <= 4, "gemv: %d weights (1..4)", c.nw);
  XTG_CHECK(c.m >= 1 && c.m <= kMaxRows, "gemv: %d rows (1..%d)", c.m, kMaxRows);
  XTG_CHECK(raw_kind(c) || c.xop, "gemv: no activations");
  GemvArgs a{};
  const int kt = c.w[0]->kt;
  for (int i = 0; i < c.nw; ++i) XTG_CHECK(c.w[i]->kt == kt, "gemv: input widths differ");
  const bool xr = raw_kind(c);
  XTG_CHECK(c.ksplit == 1 || (c.ksplit == 2 && !xr && c.m >= 2 && c.y_part > 0),
            "gemv: a K split takes a prepared operand of 2..8 rows and a second output set");
  const int ks = c.ksplit;
  GemvShape sh = call_shape(c);
  if (ks == 2) {
    // half of K, two row-blocks per wave (down / o / gate 3072..8192 wide at 8 rows, measured on MI355X: 1.7 / 0.6 /
    // 1.5 us per launch faster than the whole K, against 0.4 us slower / no gain at one row-block)
    int nbs[4];
    for (int i = 0; i < c.nw; ++i) nbs[i] = c.w[i]->nb;
    sh = gemv_shape((kt + 1) / 2, nbs, c.nw, c.m, false);
    if (shape_ok(2, sh.t, sh.s)) sh.r = 2;
  }
  int wgs = 0;
  for (int i = 0; i < c.nw; ++i) {
    a.tiles[i] = c.w[i]->tiles;
    a.nb[i] = c.w[i]->nb;
    a.n[i] = c.w[i]->n;
    a.global[i] = c.w[i]->global;
    a.y_off[i] = (long long)c.y_off[i];
    a.col_scale[i] = c.col_scale[i];
    wgs += (c.w[i]->nb + sh.r - 1) / sh.r;
    a.wg_end[i] = wgs;
  }
  for (int i = c.nw; i < 4; ++i) a.wg_end[i] = wgs;
  a.nw = c.nw;
  a.kt = kt;
  a.m = c.m;
  a.xop = xr ? nullptr : static_cast<const uint4*>(c.xop);
  a.xinv = xr ? nullptr : c.xinv;
  a.x = c.x;
  a.k = c.k;
  a.y = c.y;
  a.y_part = ks == 2 ? (long long)c.y_part : 0;
  a.waves = sh.s;
#ifdef XTG_PHASE_STAMPS
  a.stamps = g_stamp_buf;
  a.stamp_records = g_stamp_records;
#endif
  XTG_CHECK(sh.s * sh.t * ks >= kt && sh.s <= 16, "gemv: shape R=%d T=%d S=%d for %d k-tiles", sh.r, sh.t, sh.s, kt);
  const int threads = sh.s * 64;
  GemvFn mx = xr && c.m <= 2 && mx_enabled() ? gemv_mx_fn(sh.r, sh.t, threads, c.m) : nullptr;
  GemvFn fn = mx ? mx : gemv_fn(sh.r, sh.t, threads, xr);
  XTG_CHECK(fn != nullptr, "gemv: no kernel for shape R=%d T=%d%s", sh.r, sh.t, xr ? " on raw rows" : "");
  const size_t lds = (sh.s > 1 ? size_t(sh.s) * size_t(sh.r) * kMaxRows * 4 * sizeof(f32x4) : 0) +
                     (xr ? size_t(sh.s) * (mx ? kMxStageVecs : kStageVecs) * sizeof(uint4) : 0);
  allow_lds(reinterpret_cast<const void*>(fn), lds);
  hipLaunchKernelGGL(fn, dim3(unsigned(wgs), unsigned(ks)), dim3(unsigned(threads)), lds, stream, a);
  HIP_CHECK(hipGetLastError());
  const int mt = threads <= 512 ? 512 : 1024;
  if (mx) return strf("gemv_mx_kernel<%d, %d, %d, %d>", sh.r, sh.t, mt, c.m);
  if (xr) return strf("gemv_kernel<%d, %d, %d, bf16>", sh.r, sh.t, mt);
  return ks == 2 ? strf("gemv_kernel<%d, %d, %d> (K / 2)", sh.r, sh.t, mt) : strf("gemv_kernel<%d, %d, %d>", sh.r, sh.t, mt);
}

}  // namespace xtg::hip

// ----------------------------------------------------------------------------- fused decode-step projections

namespace xtg::hip {

struct FusedArgs {
  GemvArgs g;
  int in_groups;
  const float* in_x;
  const float* in_o;
  const float* in_lr;
  const float* in_part;
  float* in_xout;
  float in_ia, in_ib;
  int in_post;
  const float* out_x;
  const float* out_lr;
  const float* out_sg;
  const float* out_su;
  float* out_part;
  _Float16* out_op;
  float out_ea, out_eb;
};

// Unit rows take the operand exponent 2^14 (|x| <= 1 keeps |x 2^14| below f16's maximum).
constexpr float kRowsUp = 16384.f, kRowsDown = 1.f / 16384.f;

// LDS of a fused launch, in floats: each wave's high + low column sums [S][R][NCP column pairs][4 gg][4 e] (NCP:
// 2 for kInSlerp's a and b, else 1), their totals over the waves [R][NCP][16], then each wave's staging of one
// k-tile's live operand columns [S][4 steps][8 entries][8 f16].
struct FusedLds {
  int red, sums, stage, total;
  __host__ __device__ FusedLds(int S, int R, int in) {
    const int ncp = in == kInSlerp ? 2 : 1;
    red = 0;
    sums = red + S * R * ncp * 16;   // then the waves' totals, [R][NCP][16]
    stage = sums + R * ncp * 16;
    total = stage + (in == kInNorm ? S * 128 : 0);
  }
};

// A work-group barrier for LDS only: the waves' LDS writes are complete and visible after it, but their outstanding
// global loads are not waited for (__syncthreads' fence waits for every vector memory operation, so loads issued
// just before it for the epilogue would hold the whole work-group).
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The row values one lane reads for the kInNorm operand of a k-tile: inputs l and l + 64 of the tile; indices
// clamped into the row, so every load is issued before anything waits.
struct TileRow {
  float x[2];
};

__device__ inline void load_row(const FusedArgs& f, int k, int kt, bool kt_ok, int lane, TileRow& r) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kg = kt * kTileK + lane + 64 * h;
    r.x[h] = f.in_x[kt_ok && kg < k ? kg : 0];
  }
}

// One k-tile's kInNorm operand (h r) from the row into a wave's staging area, in operand order (input kk of column
// c at step (kk / 8) % 4, entry 4 c + kk / 32, element kk % 8; the 8 entries of the two live columns per step).
__device__ inline void stage_row(int k, int kt, bool kt_ok, int lane, float r_fac, const TileRow& r,
                                 _Float16* st16) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kk = lane + 64 * h, kg = kt * kTileK + kk;
    const bool valid = kt_ok && kg < k;
    float v = r.x[h] * r_fac;
    v = valid ? v : 0.f;
    const float sc = v * kRowsUp;
    const _Float16 hi = (_Float16)sc;
    const _Float16 lo = (_Float16)(sc - (float)hi);
    const int g = kk >> 5, t = (kk >> 3) & 3, e8 = kk & 7;
    st16[(t * 8 + g) * 8 + e8] = hi;       // column 0: entry g
    st16[(t * 8 + 4 + g) * 8 + e8] = lo;   // column 1: entry 4 + g
  }
}

// The GEMV of gemv_kernel (prepared-operand form) for one activation row with the fused input and output sides of
// kernels.hpp. The row's factors come from the producer's P records, laid out [Q][P]: a wave adds them
// lane-strided, then across its lanes (the same order in every wave and work-group: identical factors). kInNorm
// needs them before its math (every wave makes them itself, so the launch has no barrier before its math);
// kInSlerp only in the epilogue, where wave 0 makes them. Every global load the launch needs goes out first, the
// L2-resident ones (records, row values, epilogue inputs) ahead of the weights from HBM (a wave's loads retire in
// order), and none behind a branch (the compiler's wait counts after a branch assume its loads were not issued).
// Every thread reaches every barrier. Two k-tiles per wave (K <= 4096, at most 16 waves) is kept to 80 registers,
// so two work-groups of 12 waves (K = 3072) share a CU: the decode step's projections of 320 and 512 work-groups
// then run in one round over the 256 CUs.
template <int R, int T, int MAXT, int IN, int OUT>
__global__ void __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(T == 2 ? 6 : 1)))
gemv_fused_kernel(const FusedArgs f) {
  const GemvArgs& a = f.g;
  extern __shared__ f32x4 red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, S = a.waves;
  constexpr bool PAIR = OUT == kOutSwiglu;
  constexpr int RB = PAIR ? R / 2 : R;   // row-blocks per weight: PAIR takes RB of gate and the same RB of up
  static_assert(!PAIR || R % 2 == 0, "paired row-blocks");
  constexpr bool RECS = IN != kInOp;          // factors from the producer's records
  constexpr bool STAGE = IN == kInNorm;       // the operand built from the row in the prologue
  constexpr int Q = IN == kInSlerp ? 5 : 1;   // quantities per record (input side)
  constexpr int NI = Q == 5 ? 3 : 8;          // records per quantity a lane holds from the start (P <= 64 NI)
  int wi = 0;
  if constexpr (!PAIR)
    while (wi < 3 && int(blockIdx.x) >= a.wg_end[wi]) ++wi;   // wg_end past the last weight = the total
  const int rb0 = (int(blockIdx.x) - (wi ? a.wg_end[wi - 1] : 0)) * RB;
  const int KT = a.kt, kt0 = wave * T;
  const FusedLds L(S, R, IN);
  float* ldsf = reinterpret_cast<float*>(red);

  const int col = lane & 15, grp = lane >> 4;
  // the live operand columns: the row's high and low parts; kInSlerp: those of a (0, 1) and of b (2, 3)
  const bool live_col = col < (IN == kInSlerp ? 4 : 2);
  const int entry = 4 * col + grp;
  const int P = f.in_groups;
  // the records through a buffer resource: a load past them returns zero
  const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(f.in_part), (short)0, RECS ? Q * P * 4 : 0, 0x00020000);
  auto record = [&](int q, int p) {
    const uint32_t off = p < P ? uint32_t((q * P + p) * 4) : 0x80000000u;
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rres, int(off), 0, 0));
  };
  float rv[RECS ? Q : 1][RECS ? NI : 1];
  TileRow rows[STAGE ? T : 1];
  // kInNorm makes its factor before its math: the records and the row go out first
  if constexpr (STAGE) {
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int i = 0; i < NI; ++i) rv[q][i] = record(q, lane + 64 * i);
#pragma unroll
    for (int u = 0; u < T; ++u) load_row(f, a.k, kt0 + u, kt0 + u < KT, lane, rows[u]);
  }
  uint4 xb[T][4];
  uint4 cw[T][R];
  uint32_t sw[T][R];
  // the prepared operand through a buffer resource (zero past it: k-tiles past k, columns past the row)
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4*>(a.xop), (short)0, STAGE ? 0 : KT * 4096, 0x00020000);
#pragma unroll
  for (int u = 0; u < T; ++u) {
    const int kt = kt0 + u;
    const bool ok = kt < KT;
    if constexpr (!STAGE) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t off = ok && live_col ? uint32_t(((kt * 4 + t) * 64 + entry) * 16) : 0x80000000u;
        xb[u][t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, int(off), 0, 0));
      }
    }
    // an absent weight tile (past the last row-block or past k) loads a tile of the same weight, clamped: past
    // the last row-block its results are not stored, past k its products meet zero operand columns
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int w = PAIR ? (r < RB ? 0 : 1) : wi;
      const int b = rb0 + (PAIR && r >= RB ? r - RB : r);
      const int bc = b < a.nb[w] ? b : a.nb[w] - 1, ktc = ok ? kt : KT - 1;
      const uint8_t* tile = a.tiles[w] + (size_t(bc) * size_t(KT) + size_t(ktc)) * kTileBytes;
      const u32x4 c4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + 16 * lane));
      cw[u][r] = make_uint4(c4[0], c4[1], c4[2], c4[3]);
      sw[u][r] = uint32_t(__builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(tile + 1024 + 2 * lane)));
    }
  }

  // the row's factors from the records: fa, fb, f2 (kInSlerp; with in_post's norm folded into f2) or r (kInNorm, in
  // fac[0])
  auto factors = [&](float (&fac)[3]) {
    float sq[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) v += rv[q][i];
      for (int p0 = 64 * NI; p0 < P; p0 += 64) v += record(q, p0 + lane);
      sq[q] = wave_sum(v);
    }
    fac[0] = inv_norm_of(sq[0]);
    fac[1] = fac[2] = 0.f;
    if constexpr (IN == kInSlerp) {
      fac[1] = inv_norm_of(sq[1]);
      const float t2 = fac[0] * fac[0] * sq[2] + 2.f * fac[0] * fac[1] * sq[3] + fac[1] * fac[1] * sq[4];
      fac[2] = inv_norm_of(t2);
      if (f.in_post != kPostNone) {
        const float x2 = fac[2] * fac[2] * t2;   // sum x_new^2
        fac[2] *= f.in_post == kPostAddNorm ? 2.f * inv_norm_of(4.f * x2) : inv_norm_of(x2);
      }
    }
  };
  if constexpr (STAGE) {
    float fac[3];
    factors(fac);
    _Float16* st16 = reinterpret_cast<_Float16*>(ldsf + L.stage) + size_t(wave) * 256;
    const uint4* st4 = reinterpret_cast<const uint4*>(st16);
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const int kt = kt0 + u;
      stage_row(a.k, kt, kt < KT, lane, fac[0], rows[u], st16);
      wave_lds_order();
#pragma unroll
      for (int t = 0; t < 4; ++t) xb[u][t] = live_col ? st4[t * 8 + entry] : make_uint4(0, 0, 0, 0);
      wave_lds_order();
    }
  }

  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < T; ++u) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f16x2 s0 = scale_pair(sw[u][r], 0), s1 = scale_pair(sw[u][r], 1);
      const uint32_t words[4] = {cw[u][r].x, cw[u][r].y, cw[u][r].z, cw[u][r].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f16x8 A = dequant8(words[t], t < 2 ? s0 : s1);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(f16x8, xb[u][t]), acc[r], 0, 0, 0);
      }
    }
  }

  // Wave 0 loads what only the epilogue needs now, while the other waves finish: the records (kInSlerp), the
  // x_new elements' inputs (work-group j writes its share of the row) and this thread's output's sg, su (PAIR)
  // or x, lr (slerp).
  const int xn_per = (a.k + int(gridDim.x) - 1) / int(gridDim.x), xn0 = int(blockIdx.x) * xn_per;
  float sx = 0.f, so = 0.f, sl = 0.f, ep_a = 0.f, ep_b = 0.f;
  if (wave == 0) {
    if constexpr (IN == kInSlerp) {
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int i = 0; i < NI; ++i) rv[q][i] = record(q, lane + 64 * i);
      const int kc = lane < xn_per && xn0 + lane < a.k ? xn0 + lane : 0;
      sx = f.in_x[kc];
      so = f.in_o[kc];
      sl = f.in_lr[kc];
    }
    if constexpr (OUT != kOutPlain) {
      const int b = rb0 + (int(threadIdx.x) >> 4), w0 = PAIR ? 0 : wi;
      const int o_i = b * kTileRows + (int(threadIdx.x) & 15), n = a.n[w0];
      const int oc = int(threadIdx.x) < RB * 16 && o_i < n ? o_i : 0;
      ep_a = PAIR ? f.out_sg[oc] : f.out_x[oc];
      ep_b = PAIR ? f.out_su[oc] : f.out_lr[oc];
    }
  }
  // Each wave adds its high and low columns (lanes l and l ^ 1) and stores the column pairs' sums; then the first
  // RB * 16 threads (all in wave 0) add the waves' sums in a fixed order, one output each: row 4 gg + e of
  // row-block r (of each weight, PAIR), i = 16 r + 4 gg + e; then the work-group's record, each quantity added over
  // those threads by wave_sum.
  constexpr int NCP = IN == kInSlerp ? 2 : 1;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    f32x4 v = acc[r];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += dpp<kDppXor1>(v[e]);
    const int c = lane & 15;
    if ((c & 1) == 0 && c < 2 * NCP)
      *reinterpret_cast<f32x4*>(ldsf + (((wave * R + r) * NCP + (c >> 1)) * 4 + (lane >> 4)) * 4) = v;
  }
  // kInSlerp: y = global (f2 fa 2^-ea (W a) + f2 fb 2^-eb (W b)), and this work-group's share of x_new; wave 0
  // works them out before the barrier, while the other waves may still be loading
  float ca = 0.f, cb = 0.f;
  if constexpr (IN == kInSlerp) {
    if (wave == 0) {
      float fac[3];
      factors(fac);
      ca = fac[2] * fac[0] * f.in_ia;
      cb = fac[2] * fac[1] * f.in_ib;
      if (f.in_xout && lane < xn_per && xn0 + lane < a.k) {
        const float ya = sx * fac[0], yb = so * fac[1];
        f.in_xout[xn0 + lane] = (ya + sl * (yb - ya)) * fac[2];
      }
    }
  }
  lds_barrier();
  if (wave != 0) return;
  // the waves' sums added in wave order, one (row-block, column pair, row) per lane
  float* tot = ldsf + L.sums;
  for (int u = lane; u < R * NCP * 16; u += 64) {
    const int rr = u / (NCP * 16), cp = (u / 16) % NCP, gg = (u >> 2) & 3, e = u & 3;
    const float* p = ldsf + ((rr * NCP + cp) * 4 + gg) * 4 + e;
    float sum = 0.f;
#pragma unroll
    for (int w0 = 0; w0 < 16; w0 += 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = p[(w0 + i < S ? w0 + i : S - 1) * R * NCP * 16];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (w0 + i < S) sum += v[i];
    }
    tot[u] = sum;
  }
  wave_lds_order();   // the totals are in
  float q[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  if (int(threadIdx.x) < RB * 16) {
    const int r = int(threadIdx.x) >> 4, gg = (int(threadIdx.x) >> 2) & 3, e = int(threadIdx.x) & 3;
    const int b = rb0 + r, w0 = PAIR ? 0 : wi, n = a.n[w0], o_i = b * kTileRows + 4 * gg + e;
    // accumulator row 4 gg + e of row-block rr: column pair cp's total over the waves
    auto pair_sum = [&](int rr, int cp) { return tot[(rr * NCP + cp) * 16 + 4 * gg + e]; };
    auto sum_of = [&](int rr) {
      if constexpr (IN == kInSlerp)
        return ca * pair_sum(rr, 0) + cb * pair_sum(rr, 1);
      else
        return pair_sum(rr, 0) * (IN == kInOp ? (a.xinv ? a.xinv[0] : 1.f) : kRowsDown);
    };
    if (b < a.nb[w0] && o_i < n) {
      float* yp = a.y + a.y_off[w0];
      if constexpr (PAIR) {
        const float z = (sum_of(r) * a.global[0]) * ep_a;
        const float hv = z / (1.f + expf(-z)) * ((sum_of(r + RB) * a.global[1]) * ep_b);
        yp[o_i] = hv;
        q[0] = hv * hv;
      } else {
        const float* cs = a.col_scale[wi];
        const float sv = sum_of(r) * a.global[wi];
        const float o = cs ? sv * cs[o_i] : sv;
        yp[o_i] = o;
        if constexpr (OUT == kOutSlerp) {
          const float x = ep_a, lr = ep_b, ol = 1.f - lr;
          q[0] = x * x;
          q[1] = o * o;
          q[2] = (ol * ol) * (x * x);
          q[3] = (ol * lr) * (x * o);
          q[4] = (lr * lr) * (o * o);
          if (f.out_op) {
            // the consumer's operand in the linear form of the slerp: a = (1 - lr) x at 2^ea, b = lr o at 2^eb,
            // high and low f16 parts in columns 0, 1 (a) and 2, 3 (b) of input o_i
            const int kt = o_i >> 7, kk = o_i & 127, t = (kk >> 3) & 3, g = kk >> 5, e8 = kk & 7;
            _Float16* op = f.out_op + size_t((kt * 4 + t) * 64 + g) * 8 + size_t(e8);
            const float av = ol * x * f.out_ea, bv = lr * o * f.out_eb;
            const _Float16 ah = (_Float16)av, bh = (_Float16)bv;
            op[0] = ah;
            op[4 * 8] = (_Float16)(av - (float)ah);
            op[8 * 8] = bh;
            op[12 * 8] = (_Float16)(bv - (float)bh);
          }
        }
      }
    }
  }
  if constexpr (OUT != kOutPlain) {
    constexpr int QO = OUT == kOutSlerp ? 5 : 1;
#pragma unroll
    for (int i = 0; i < QO; ++i) {
      const float t = wave_sum(q[i]);
      if (lane == 0) f.out_part[size_t(i) * gridDim.x + blockIdx.x] = t;
    }
  }
}

namespace {
using FusedFn = void (*)(const FusedArgs);

template <int R, int T, int IN, int OUT>
FusedFn fused_pick(int threads) {
  return threads <= 512 ? gemv_fused_kernel<R, T, 512, IN, OUT> : gemv_fused_kernel<R, T, 1024, IN, OUT>;
}

// the combinations the decode step makes: qkvg (slerp rows in), gate / up (slerp rows in, SwiGLU out), down (norm
// rows in, slerp records out), o (prepared operand in, slerp records out); R row-blocks (per weight when paired);
// two k-tiles per wave up to K = 4096, four above (the plain GEMV's k-split)
FusedFn fused_fn(int r, int t, int threads, int in, int out) {
#define XTG_F(R, T, IN, OUT) \
  if (r == R && t == T && in == IN && out == OUT) return fused_pick<R, T, IN, OUT>(threads);
  XTG_F(1, 2, kInSlerp, kOutPlain) XTG_F(2, 2, kInSlerp, kOutPlain) XTG_F(4, 2, kInSlerp, kOutPlain)
  XTG_F(2, 2, kInSlerp, kOutSwiglu) XTG_F(4, 2, kInSlerp, kOutSwiglu) XTG_F(2, 2, kInOp, kOutSwiglu)
  XTG_F(1, 2, kInNorm, kOutSlerp) XTG_F(2, 2, kInNorm, kOutSlerp) XTG_F(1, 4, kInNorm, kOutSlerp)
  XTG_F(1, 2, kInOp, kOutSlerp) XTG_F(2, 2, kInOp, kOutSlerp) XTG_F(1, 4, kInOp, kOutSlerp)
  XTG_F(1, 4, kInSlerp, kOutPlain) XTG_F(2, 4, kInSlerp, kOutSwiglu)
#undef XTG_F
  return nullptr;
}

// The launch shape: the plain GEMV's k-split (so a fused projection sums every output in the order the plain
// launch does), T k-tiles of 2 or 4 (the fused kernels are made for those); the row-blocks as the plain GEMV picks
// them, at least one pair when paired.
GemvShape fused_shape(const FusedGemv& f) {
  int nbs[4];
  for (int i = 0; i < f.c.nw; ++i) nbs[i] = f.c.w[i]->nb;
  GemvShape sh = gemv_shape(f.c.w[0]->kt, nbs, f.c.nw, f.c.m, false);
  if (f.out == kOutSwiglu) sh.r = sh.r >= 4 ? 4 : 2;   // one or two pairs
  if (f.out == kOutSlerp || f.in == kInNorm) sh.r = std::min(sh.r, 2);
  if (sh.t != 2 && sh.t != 4) {   // a k-split the fused kernels are not made for (a wide head's three k-tiles)
    sh.t = f.c.w[0]->kt <= 32 ? 2 : 4;
    sh.s = (f.c.w[0]->kt + sh.t - 1) / sh.t;
    sh.r = std::min(sh.r, 4);
  }
  return sh;
}
}  // namespace

int fused_gemv_groups(const FusedGemv& f) {
  const GemvShape sh = fused_shape(f);
  if (f.out == kOutSwiglu) return (f.c.w[0]->nb + sh.r / 2 - 1) / (sh.r / 2);
  int wgs = 0;
  for (int i = 0; i < f.c.nw; ++i) wgs += (f.c.w[i]->nb + sh.r - 1) / sh.r;
  return wgs;
}

std::string fused_gemv_unsupported(const FusedGemv& f) {
  const GemvCall& c = f.c;
  if (c.nw < 1 || c.nw > 4) return strf("%d weights (1..4)", c.nw);
  if (c.m != 1) return strf("%d rows (one)", c.m);
  const int kt = c.w[0]->kt;
  for (int i = 0; i < c.nw; ++i)
    if (c.w[i]->kt != kt) return "input widths differ";
  if (f.out == kOutSwiglu && (c.nw != 2 || c.w[0]->n != c.w[1]->n)) return "SwiGLU pairs two weights of one shape";
  if (f.out == kOutSlerp && c.nw != 1) return "slerp records come from one weight";
  if (f.in != kInOp && (f.in_groups < 1 || f.in_groups > kMaxFusedGroups))
    return strf("records of %d work-groups (1..%d)", f.in_groups, kMaxFusedGroups);
  const GemvShape sh = fused_shape(f);
  if (sh.t != 2 && sh.t != 4) return strf("%d k-tiles per wave (2 or 4)", sh.t);
  if (sh.s > 16 || sh.s * sh.t < kt)
    return strf("%d k-tiles at %d per wave need %d waves (at most 16)", kt, sh.t, (kt + sh.t - 1) / sh.t);
  const int wgs = fused_gemv_groups(f);
  if (f.in == kInSlerp && (c.k + wgs - 1) / wgs > 64)
    return strf("x_new of %d inputs over %d work-groups (at most 64 each)", c.k, wgs);
  if (f.out != kOutPlain && wgs > kMaxFusedGroups)
    return strf("%d work-groups' records (at most %d)", wgs, kMaxFusedGroups);
  if (!fused_fn(sh.r, sh.t, sh.s * 64, f.in, f.out))
    return strf("no kernel for R=%d T=%d (in %d, out %d)", sh.r, sh.t, f.in, f.out);
  return std::string();
}

std::string launch_gemv_fused(const FusedGemv& f, hipStream_t stream) {
  const GemvCall& c = f.c;
  const std::string why = fused_gemv_unsupported(f);
  XTG_CHECK(why.empty(), "fused gemv: %s", why.c_str());
  XTG_CHECK(f.in == kInNorm || c.xop, "fused gemv: no operand");
  XTG_CHECK(f.in == kInOp || (f.in_x && f.in_part && c.k > 0 && c.k % 16 == 0 && (f.in == kInNorm || (f.in_o && f.in_lr))),
            "fused gemv: rows, records and width for the input side");
  XTG_CHECK(f.out != kOutSwiglu || (f.out_sg && f.out_su && f.out_part), "fused gemv: SwiGLU scales and records");
  XTG_CHECK(f.out != kOutSlerp || (f.out_x && f.out_lr && f.out_part && !c.col_scale[0]),
            "fused gemv: slerp rows and records");
  FusedArgs a{};
  const int kt = c.w[0]->kt;
  const GemvShape sh = fused_shape(f);
  const int rb = f.out == kOutSwiglu ? sh.r / 2 : sh.r;
  int wgs = 0;
  for (int i = 0; i < c.nw; ++i) {
    a.g.tiles[i] = c.w[i]->tiles;
    a.g.nb[i] = c.w[i]->nb;
    a.g.n[i] = c.w[i]->n;
    a.g.global[i] = c.w[i]->global;
    a.g.y_off[i] = (long long)c.y_off[i];
    a.g.col_scale[i] = c.col_scale[i];
    if (f.out != kOutSwiglu || i == 0) wgs += (c.w[i]->nb + rb - 1) / rb;
    a.g.wg_end[i] = wgs;
  }
  for (int i = c.nw; i < 4; ++i) a.g.wg_end[i] = wgs;
  a.g.nw = c.nw;
  a.g.kt = kt;
  a.g.m = c.m;
  a.g.xop = static_cast<const uint4*>(c.xop);
  a.g.xinv = c.xinv;
  a.g.k = c.k;
  a.g.y = c.y;
  a.g.waves = sh.s;
  a.in_groups = f.in_groups;
  a.in_x = f.in_x;
  a.in_o = f.in_o;
  a.in_lr = f.in_lr;
  a.in_part = f.in_part;
  a.in_xout = f.in_xout;
  a.in_ia = f.in_ia;
  a.in_ib = f.in_ib;
  a.in_post = f.in_post;
  a.out_op = static_cast<_Float16*>(f.out_op);
  a.out_ea = f.out_ea;
  a.out_eb = f.out_eb;
  a.out_x = f.out_x;
  a.out_lr = f.out_lr;
  a.out_sg = f.out_sg;
  a.out_su = f.out_su;
  a.out_part = f.out_part;
  XTG_CHECK(wgs == fused_gemv_groups(f), "fused gemv: %d work-groups", wgs);
  const int threads = sh.s * 64;
  FusedFn fn = fused_fn(sh.r, sh.t, threads, f.in, f.out);
  const size_t lds = size_t(FusedLds(sh.s, sh.r, f.in).total) * sizeof(float);
  allow_lds(reinterpret_cast<const void*>(fn), lds);
  hipLaunchKernelGGL(fn, dim3(unsigned(wgs)), dim3(unsigned(threads)), lds, stream, a);
  HIP_CHECK(hipGetLastError());
  static const char* kIn[] = {"op", "slerp", "norm"};
  static const char* kOut[] = {"plain", "slerp", "swiglu"};
  return strf("gemv_fused_kernel<%d, %d, %d, %s, %s>", sh.r, sh.t, threads <= 512 ? 512 : 1024, kIn[f.in],
              kOut[f.out]);
}

}  // namespace xtg::hip

#ifdef XTG_PHASE_STAMPS
// The phase-stamp build's one extra export: every later gemv_kernel launch writes its records into buf (device
// memory of records * 64 bytes; NULL: none); *clock_khz receives the rate of the clock the stamps read.
extern "C" int xtg_hip_phase_stamps(void* buf, long long records, int* clock_khz) {
  xtg::hip::g_stamp_buf = static_cast<unsigned long long*>(buf);
  xtg::hip::g_stamp_records = buf ? records : 0;
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return -1;
  *clock_khz = khz;
  return 0;
}
#endif
