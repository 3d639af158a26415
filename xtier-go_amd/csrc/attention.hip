// Decode attention over a device-resident KV cache, and the cache's store.
//
// Semantics (engine/src/kv.cpp:166-286, npu/xtg_npu.cpp:236-258): query row i of this call (position pos0 + i)
// attends, for each of its q heads, to the cached keys whose stored position q satisfies 0 <= q < pos0 and
// (window <= 0 or pos0 + i - q < window), and to this call's own keys j <= i (with i - j < window); FP32 softmax of
// scale * q.k. For a linear cache the stored position of slot s is s; for a ring it is whatever position was last
// written there (the slot-position array), so the mask is rebuilt from slot positions on every call.
//
// Device cache layout (head-major, in matrix-core operand order, slots padded to a multiple of 32):
//   K: per head, per block of 16 slots, per 32-wide chunk c of head_dim: 64 lanes x 8 BF16, lane (g, i) holding
//      slot 16 b + i, dims 32 c + 8 g .. +8: the A operand of v_mfma_f32_16x16x32_bf16 (keys x dims).
//   V: per head, per tile of 32 slots, per 16-wide block dd of head_dim: 64 lanes x 8 BF16, lane (g, i) holding
//      dim 16 dd + i of slots {4 g .. 4 g + 3, 16 + 4 g .. 16 + 4 g + 3}: the A operand (dims x keys) of the P.V
//      product whose B operand (keys x queries) is exactly what each lane holds of the score tile's accumulator.
//   slot_pos: int32 per slot, -1 = never written.
// An FP8 cache (E4M3 codes, one FP32 scale per (slot, head): kv.cpp:94-108) keeps the same operand order with one
// byte per element, two operands per 16-byte lane load:
//   K: per head, per block of 16 slots, per pair of 32-wide chunks: 64 lanes x 16 bytes, bytes 0..7 of lane (g, i)
//      the BF16 layout's entry for chunk 2 cp, bytes 8..15 for chunk 2 cp + 1.
//   V: per head, per tile of 32 slots, per pair of 16-wide blocks: 64 lanes x 16 bytes likewise.
//   kscale / vscale: FP32 [head][slot]. Codes become BF16 exactly (v_cvt_scalef32_pk_bf16_fp8 with scale 1); the
//   key scale multiplies the scores, the value scale the softmax weights of the P.V product (not their sum).
//
// Work (flash decoding, partials laid out as AttnPlan says):
//   attn_scan_kernel: a work-group of 4 waves per (KV head, split of the key tiles). Scores S^T = K Q^T with the q
//     vectors (times scale) split into three BF16 terms (about 24 significant bits, so sharp softmaxes keep
//     FP32-level scores); K is BF16 and exact. P.V with P split into two BF16 terms. The q heads sharing a KV head
//     and the query rows are stacked as MFMA columns (q-col = row * group + head), so every K and V byte is read
//     once per KV head. Each wave streams its tiles with the next tile's loads in flight; the waves' states are
//     merged in LDS into one partial per q-col.
//   Own keys (FP32, not rounded to the cache's BF16), one more partial: for the attention call, FP32 MFMA over
//     tiles of 16 q-cols x 16 keys (attn_own_mfma_kernel); inside the decode step's producer (qk_produce_kernel),
//     one wave per q-col on the vector ALUs.
//   attn_merge_kernel / attn_gate_kernel: one work-group per query row merges its partials (kv.cpp:262-285);
//     the gate variant applies the decode step's sigmoid gate and norm and writes the o-projection's operand.
#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

#include "attention.hpp"
#include "common.hpp"
#include "rowops.hpp"

namespace xtg::hip {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;      // waves per work-group (one split)
constexpr int kTile = 32;      // slots per tile

// ------------------------------------------------------------------------------------------------ layout maths

__host__ __device__ inline size_t k_index(int h, int slot, int dim, int slots_pad, int d) {
  const int b = slot >> 4, i = slot & 15, c = dim >> 5, g = (dim & 31) >> 3, e = dim & 7;
  return ((((size_t(h) * size_t(slots_pad >> 4) + size_t(b)) * size_t(d >> 5) + size_t(c)) * 64 + size_t(g * 16 + i)) * 8) +
         size_t(e);
}

__host__ __device__ inline size_t v_index(int h, int slot, int dim, int slots_pad, int d) {
  const int t = slot >> 5, kk = slot & 31;
  const int half = kk >> 4, r = kk & 15;   // key 16 half + 4 g + (e & 3)
  const int g = r >> 2, e = half * 4 + (r & 3);
  const int dd = dim >> 4, i = dim & 15;
  return ((((size_t(h) * size_t(slots_pad >> 5) + size_t(t)) * size_t(d >> 4) + size_t(dd)) * 64 + size_t(g * 16 + i)) * 8) +
         size_t(e);
}

__host__ __device__ inline size_t k8_index(int h, int slot, int dim, int slots_pad, int d) {
  const int b = slot >> 4, i = slot & 15, c = dim >> 5, g = (dim & 31) >> 3, e = dim & 7;
  return ((((size_t(h) * size_t(slots_pad >> 4) + size_t(b)) * size_t(d >> 6) + size_t(c >> 1)) * 64 +
           size_t(g * 16 + i)) * 16) + size_t((c & 1) * 8 + e);
}

__host__ __device__ inline size_t v8_index(int h, int slot, int dim, int slots_pad, int d) {
  const int t = slot >> 5, kk = slot & 31;
  const int half = kk >> 4, r = kk & 15;
  const int g = r >> 2, e = half * 4 + (r & 3);
  const int dd = dim >> 4, i = dim & 15;
  return ((((size_t(h) * size_t(slots_pad >> 5) + size_t(t)) * size_t(d >> 5) + size_t(dd >> 1)) * 64 +
           size_t(g * 16 + i)) * 16) + size_t((dd & 1) * 8 + e);
}

size_t kv_k_index(int h, int slot, int dim, int slots_pad, int d) { return k_index(h, slot, dim, slots_pad, d); }
size_t kv_v_index(int h, int slot, int dim, int slots_pad, int d) { return v_index(h, slot, dim, slots_pad, d); }
size_t kv_k8_index(int h, int slot, int dim, int slots_pad, int d) { return k8_index(h, slot, dim, slots_pad, d); }
size_t kv_v8_index(int h, int slot, int dim, int slots_pad, int d) { return v8_index(h, slot, dim, slots_pad, d); }

__device__ inline uint16_t f32_to_bf16_bits(float f) {
  // round to nearest even; a NaN stays a quiet NaN (engine/include/xtg/fp.h:18-24)
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return uint16_t((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

__device__ inline float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// The cache's E4M3 rounding (engine/src/kv.cpp:19-40): below 2^-6 the value counts subnormal steps of 2^-9 (ties
// to even); above, the FP32 mantissa is rounded to 3 bits (ties to even) and rebiased, capped at 0x7e (448); NaN
// gives 0x7f with the sign.
__device__ inline uint32_t e4m3_code(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 24) & 0x80u, a = bits & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  uint32_t code;
  if (a < 0x3c800000u) {
    const float t = __uint_as_float(a) * 512.f;   // exact: a power-of-two factor below the overflow range
    const float lo = floorf(t);
    const float frac = t - lo;                    // exact
    code = uint32_t(lo);
    code += (frac > 0.5f || (frac == 0.5f && (code & 1u))) ? 1u : 0u;
  } else {
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
    code = code > 0x7eu ? 0x7eu : code;
  }
  return sign | code;
}

// One row of D values held by a wave (lane l: dims l + 64 u) into an FP8 cache: scale amax / 448 (1 for an
// all-zero row), codes of value / scale (kv.cpp:94-108). Every lane of the wave must be active.
template <int D>
__device__ inline void store_fp8_row(const float (&x)[D / 64], uint8_t* __restrict__ c8, float* __restrict__ scl,
                                     bool is_v, int h, int slot, int slots_pad) {
  const int lane = threadIdx.x & 63;
  float am = 0.f;
#pragma unroll
  for (int u = 0; u < D / 64; ++u) am = fmaxf(am, fabsf(x[u]));
  am = wave_max(am);
  const float sc = am > 0.f ? am / 448.f : 1.f;
  const float inv = 1.f / sc;
#pragma unroll
  for (int u = 0; u < D / 64; ++u) {
    const int dim = lane + 64 * u;
    const size_t at = is_v ? v8_index(h, slot, dim, slots_pad, D) : k8_index(h, slot, dim, slots_pad, D);
    c8[at] = uint8_t(e4m3_code(x[u] * inv));
  }
  if (lane == 0) scl[size_t(h) * size_t(slots_pad) + size_t(slot)] = sc;
}

// ------------------------------------------------------------------------------------------------------ store

// One thread per (row, head, dim) of the rows kept (a ring keeps the last `slots` rows of a long call:
// engine/src/kv.cpp:75-80); slot_pos is written by the dim-0 thread of head 0.
__global__ void __launch_bounds__(256) kv_store_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                       uint16_t* __restrict__ ck, uint16_t* __restrict__ cv,
                                                       int* __restrict__ slot_pos, long long pos, int first, int n,
                                                       int kv_heads, int d, long long slots, int ring, int slots_pad) {
  const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long per_row = (long long)kv_heads * d;
  const long long rows = n - first;
  if (idx >= rows * per_row) return;
  const int r = first + int(idx / per_row);
  const int rem = int(idx % per_row), h = rem / d, dim = rem % d;
  const long long p = pos + r;
  const int slot = int(ring ? p % slots : p);
  const size_t src = (size_t(r) * size_t(kv_heads) + size_t(h)) * size_t(d) + size_t(dim);
  ck[k_index(h, slot, dim, slots_pad, d)] = f32_to_bf16_bits(k[src]);
  cv[v_index(h, slot, dim, slots_pad, d)] = f32_to_bf16_bits(v[src]);
  if (h == 0 && dim == 0) slot_pos[slot] = int(p);
}

// FP8: one wave per (row kept, head, K or V), 4 waves per work-group; slot_pos by the first wave of each row.
template <int D>
__global__ void __launch_bounds__(256) kv_store_fp8_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                           uint8_t* __restrict__ ck, uint8_t* __restrict__ cv,
                                                           float* __restrict__ ks, float* __restrict__ vs,
                                                           int* __restrict__ slot_pos, long long pos, int first,
                                                           int n, int kv_heads, long long slots, int ring,
                                                           int slots_pad) {
  const long long wv = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long long per_row = 2LL * kv_heads;
  if (wv >= (long long)(n - first) * per_row) return;   // whole waves leave together
  const int r = first + int(wv / per_row);
  const int rem = int(wv % per_row), h = rem >> 1;
  const bool is_v = rem & 1;
  const long long p = pos + r;
  const int slot = int(ring ? p % slots : p);
  const float* src = (is_v ? v : k) + (size_t(r) * size_t(kv_heads) + size_t(h)) * D;
  float x[D / 64];
#pragma unroll
  for (int u = 0; u < D / 64; ++u) x[u] = src[(threadIdx.x & 63) + 64 * u];
  store_fp8_row<D>(x, is_v ? cv : ck, is_v ? vs : ks, is_v, h, slot, slots_pad);
  if (rem == 0 && (threadIdx.x & 63) == 0) slot_pos[slot] = int(p);
}

std::string launch_kv_store(const DevKv& c, long long pos, int n, const float* k, const float* v,
                            hipStream_t stream) {
  int first = 0;
  if (c.ring && n > c.slots) first = int(n - c.slots);
  if (n - first <= 0) return std::string();
  if (c.fp8) {
    const long long waves = (long long)(n - first) * 2 * c.kv_heads;
    const dim3 grid{unsigned((waves + 3) / 4)}, block{256};
    auto* ck = static_cast<uint8_t*>(c.k);
    auto* cv = static_cast<uint8_t*>(c.v);
#define XTG_STORE8(D)                                                                                        \
  if (c.head_dim == D)                                                                                      \
    hipLaunchKernelGGL(kv_store_fp8_kernel<D>, grid, block, 0, stream, k, v, ck, cv, c.kscale, c.vscale,     \
                       c.slot_pos, pos, first, n, c.kv_heads, (long long)c.slots, c.ring ? 1 : 0, c.slots_pad);
    XTG_STORE8(64) XTG_STORE8(128) XTG_STORE8(256)
#undef XTG_STORE8
    HIP_CHECK(hipGetLastError());
    return strf("kv_store_fp8_kernel<%d>", c.head_dim);
  }
  const long long total = (long long)(n - first) * c.kv_heads * c.head_dim;
  const unsigned blocks = unsigned((total + 255) / 256);
  hipLaunchKernelGGL(kv_store_kernel, dim3(blocks), dim3(256), 0, stream, k, v, static_cast<uint16_t*>(c.k),
                     static_cast<uint16_t*>(c.v), c.slot_pos, pos, first, n, c.kv_heads, c.head_dim,
                     (long long)c.slots, c.ring ? 1 : 0, c.slots_pad);
  HIP_CHECK(hipGetLastError());
  return "kv_store_kernel";
}


// ------------------------------------------------------------------------------------------------------- scan

struct ScanArgs {
  const float* q;          // every row of the call [n_q][heads][d]
  const uint4* ck;         // cache, operand layout
  const uint4* cv;
  const int* slot_pos;
  const float* kscale;     // FP8 caches: [head][slot] scales
  const float* vscale;
  float* acc;              // the call's partials: block b's record (h, s, c) at b * blk_records + (h * splits1 + s) *
  float* ml;               // qpad + c
  size_t blk_records;
  int b0, rpb, n_q;        // work-group column y takes block b0 + y: rows (b0 + y) * rpb .. (at most rpb, below n_q)
  int heads, group, window, splits, splits1, qpad, slots_pad;
  int tile_lo, tiles;      // the key tiles to scan: tile_lo .. tile_lo + tiles - 1
  int pos0;                // positions are below 2^31 (the slot-position array is int32)
  float scale2;            // scale * log2(e)
  const float2* rope;      // raw q rows only (the decode step's fused launch): the RoPE rows [pos][d / 2]
  const float* qscale;     //   and the per-dim q scale [heads * d] (NULL: none)
  int plain;               // raw q rows used as they are (the attention call's fused launch): rope is one identity
                           //   row (cos 1, sin 0), read for every position, and no norm
};

// FP32 -> BF16 on the vector ALU (v_cvt_pk_bf16_f32, round to nearest even) and back (exact).
__device__ inline __bf16 to_bf16(float x) { return (__bf16)x; }
__device__ inline float of_bf16(__bf16 b) { return (float)b; }

// x = t0 + t1 + t2 + O(2^-24 |x|), each term the BF16 rounding of what is left.
__device__ inline void split3(const float x[8], bf16x8& t0, bf16x8& t1, bf16x8& t2) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 a = to_bf16(x[e]);
    const float r = x[e] - of_bf16(a);
    const __bf16 b = to_bf16(r);
    t0[e] = a;
    t1[e] = b;
    t2[e] = to_bf16(r - of_bf16(b));
  }
}

// Softmax weights run in the base-2 domain: scores are q.k * scale * log2(e) and every partial's max is in those
// units, so each weight is one v_exp_f32 (exp2(-inf) = 0).
constexpr float kLog2e = 1.44269504088896341f;
__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// One 32-slot tile of a KV head as a wave holds it: K as two 16-slot A operands per 32-dim chunk, V as one A
// operand per 16-dim block, and the slot positions of the lane's 8 keys.
template <int D>
struct KvTile {
  uint4 k[2][D / 32];
  uint4 v[D / 16];
  int4 p0, p1;
};

// Tile t's K operands and slot positions, and its V operands (the two halves of a tile load).
template <int D>
__device__ inline void load_tile_k(KvTile<D>& T, const uint4* __restrict__ kb, const int* __restrict__ slot_pos, int t,
                                   int lane) {
  constexpr int NC = D / 32;
  const size_t ktile = size_t(2 * NC) * 64;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int c = 0; c < NC; ++c) T.k[b][c] = kb[size_t(t) * ktile + size_t(b * NC + c) * 64 + size_t(lane)];
  const int g = lane >> 4;
  T.p0 = *reinterpret_cast<const int4*>(slot_pos + t * kTile + 4 * g);
  T.p1 = *reinterpret_cast<const int4*>(slot_pos + t * kTile + 16 + 4 * g);
}

template <int D>
__device__ inline void load_tile_v(KvTile<D>& T, const uint4* __restrict__ vb, int t, int lane) {
  constexpr int ND = D / 16;
  const size_t vtile = size_t(ND) * 64;
#pragma unroll
  for (int dd = 0; dd < ND; ++dd) T.v[dd] = vb[size_t(t) * vtile + size_t(dd) * 64 + size_t(lane)];
}

template <int D>
__device__ inline void load_tile(KvTile<D>& T, const uint4* __restrict__ kb, const uint4* __restrict__ vb,
                                 const int* __restrict__ slot_pos, int t, int lane) {
  load_tile_k<D>(T, kb, slot_pos, t, lane);
  load_tile_v<D>(T, vb, t, lane);
}

// The q operand of a scan, B of the score products: column block qb, 32-dim chunk c, BF16 term t (split3). Heads of
// more than 128 dims, and 128-dim heads in the decode step's fused launch (raw q rows), keep it in the work-group's
// LDS, where all 4 waves read it (they scan the same q-cols), as [qb][c][t][64 lanes] x 16 bytes; other scans in
// registers. For the fused launch that frees 48 registers per lane (the one-row FP8 kernel 218 -> 173): 0.7 % off
// the one-token step with BF16 caches and 1.4 % with FP8 (4K-32K, the 8-row steps 0.3-1 %), while the prefill
// scan, 16 q-cols x 2 blocks over thousands of keys, ran 10 % slower with it.
template <int D, int QB>
struct QRegs {
  bf16x8 q[QB][D / 32][3];
  __device__ bf16x8 get(int qb, int c, int t) const { return q[qb][c][t]; }
};
template <int D, int QB>
struct QLds {
  const bf16x8* base;
  int lane;
  __device__ bf16x8 get(int qb, int c, int t) const { return base[((qb * (D / 32) + c) * 3 + t) * 64 + lane]; }
};
template <int D, bool RAWQ>
constexpr bool q_in_lds() { return D > 128 || (RAWQ && D == 128); }

// The online-softmax state of the lane's column in each q-block (the same in the 4 lanes of a column).
template <int D, int QB>
struct ScanState {
  float m[QB], l[QB];
  f32x4 acc[QB][D / 16];
};

// One tile for every q-block: scores (three MFMA terms), mask, online softmax, P.V (two terms). lo[qb]: the
// lane's column sees stored positions lo .. pos0 - 1 (INT_MAX for a column with no query).
template <int D, int QB, class QS>
__device__ inline void scan_tile(const KvTile<D>& T, const QS& qop, const int (&lo)[QB], ScanState<D, QB>& st,
                                 int pos0) {
  constexpr int NC = D / 32, ND = D / 16;
  const int kpos[8] = {T.p0.x, T.p0.y, T.p0.z, T.p0.w, T.p1.x, T.p1.y, T.p1.z, T.p1.w};
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int term = 0; term < 3; ++term) {
        const bf16x8 B = qop.get(qb, c, term);   // each operand read once per tile, for both key blocks
#pragma unroll
        for (int b = 0; b < 2; ++b)
          s[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, T.k[b][c]), B, s[b], 0, 0, 0);
      }
    // mask, then the column's max over its 4 lanes x 8 keys
    float sc[8];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sc[e] = kpos[e] >= lo[qb] && kpos[e] < pos0 ? s[e >> 2][e & 3] : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = xor32_max(xor16_max(mx));
    // No branch on visibility: every lane takes part in the swaps and matrix ops below. A column with nothing
    // visible yet keeps max -inf, sum 0 and a zero accumulator (reference max 0: weights exp2(-inf) = 0).
    const float m_new = fmaxf(st.m[qb], mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float corr = exp2_fast(st.m[qb] - m_ref);
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = exp2_fast(sc[e] - m_ref);
      ps += p[e];
    }
    ps = xor32_sum(xor16_sum(ps));
    st.l[qb] = st.l[qb] * corr + ps;
    st.m[qb] = m_new;
    bf16x8 phi, plo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 h = to_bf16(p[e]);
      phi[e] = h;
      plo[e] = to_bf16(p[e] - of_bf16(h));
    }
    if (__ballot(corr != 1.f)) {   // some column's max moved: rescale (skipped once the maxima settle)
#pragma unroll
      for (int dd = 0; dd < ND; ++dd) st.acc[qb][dd] *= corr;
    }
#pragma unroll
    for (int dd = 0; dd < ND; ++dd) {
      const bf16x8 A = __builtin_bit_cast(bf16x8, T.v[dd]);
      st.acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, phi, st.acc[qb][dd], 0, 0, 0);
      st.acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, plo, st.acc[qb][dd], 0, 0, 0);
    }
  }
}

// scan_tile for BF16 heads of 128 dims or more: one tile is held, and reloaded in a skew. Once the scores have used
// this tile's K and positions, next_k(T) loads the next tile's into their registers, to land during this tile's
// softmax and P.V; once P.V has used V, next_v(T) loads the next tile's V, to land during the next scores. Each load
// then has about half a tile's work to land behind, and a wave keeps one tile's bytes in flight.
template <int D, int QB, class QS, class LK, class LV>
__device__ inline void scan_tile_skewed(KvTile<D>& T, const QS& qop, const int (&lo)[QB], ScanState<D, QB>& st,
                                        int pos0, LK&& next_k, LV&& next_v) {
  constexpr int NC = D / 32, ND = D / 16;
  f32x4 s[QB][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    s[qb][0] = s[qb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int term = 0; term < 3; ++term) {
        const bf16x8 B = qop.get(qb, c, term);
#pragma unroll
        for (int b = 0; b < 2; ++b)
          s[qb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, T.k[b][c]), B, s[qb][b], 0, 0, 0);
      }
  }
  const int kpos[8] = {T.p0.x, T.p0.y, T.p0.z, T.p0.w, T.p1.x, T.p1.y, T.p1.z, T.p1.w};
  next_k(T);
  bf16x8 phi[QB], plo[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    float sc[8];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sc[e] = kpos[e] >= lo[qb] && kpos[e] < pos0 ? s[qb][e >> 2][e & 3] : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(st.m[qb], mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float corr = exp2_fast(st.m[qb] - m_ref);
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = exp2_fast(sc[e] - m_ref);
      ps += p[e];
    }
    ps = xor32_sum(xor16_sum(ps));
    st.l[qb] = st.l[qb] * corr + ps;
    st.m[qb] = m_new;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 h = to_bf16(p[e]);
      phi[qb][e] = h;
      plo[qb][e] = to_bf16(p[e] - of_bf16(h));
    }
    if (__ballot(corr != 1.f)) {
#pragma unroll
      for (int dd = 0; dd < ND; ++dd) st.acc[qb][dd] *= corr;
    }
  }
#pragma unroll
  for (int dd = 0; dd < ND; ++dd) {
    const bf16x8 A = __builtin_bit_cast(bf16x8, T.v[dd]);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      st.acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, phi[qb], st.acc[qb][dd], 0, 0, 0);
      st.acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, plo[qb], st.acc[qb][dd], 0, 0, 0);
    }
  }
  next_v(T);
}

// The FP8 form of a tile: K as two 16-slot blocks of D / 64 lane loads (two operands each), V as D / 32 loads, the
// positions and the key and value scales of the lane's 8 keys.
template <int D>
struct KvTile8 {
  uint4 k[2][D / 64];
  uint4 v[D / 32];
  int4 p0, p1;
  float4 ks0, ks1, vs0, vs1;
};

// An FP8 tile's halves: K codes, slot positions and key scales; V codes and value scales.
template <int D>
__device__ inline void load_tile_k(KvTile8<D>& T, const uint4* __restrict__ kb, const int* __restrict__ slot_pos,
                                   const float* __restrict__ ks, int t, int lane) {
  constexpr int NP = D / 64;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int c = 0; c < NP; ++c) T.k[b][c] = kb[(size_t(2 * t + b) * NP + size_t(c)) * 64 + size_t(lane)];
  const int at = t * kTile + 4 * (lane >> 4);
  T.p0 = *reinterpret_cast<const int4*>(slot_pos + at);
  T.p1 = *reinterpret_cast<const int4*>(slot_pos + at + 16);
  T.ks0 = *reinterpret_cast<const float4*>(ks + at);
  T.ks1 = *reinterpret_cast<const float4*>(ks + at + 16);
}

template <int D>
__device__ inline void load_tile_v(KvTile8<D>& T, const uint4* __restrict__ vb, const float* __restrict__ vs, int t,
                                   int lane) {
  constexpr int NV = D / 32;
#pragma unroll
  for (int dp = 0; dp < NV; ++dp) T.v[dp] = vb[(size_t(t) * NV + size_t(dp)) * 64 + size_t(lane)];
  const int at = t * kTile + 4 * (lane >> 4);
  T.vs0 = *reinterpret_cast<const float4*>(vs + at);
  T.vs1 = *reinterpret_cast<const float4*>(vs + at + 16);
}

template <int D>
__device__ inline void load_tile(KvTile8<D>& T, const uint4* __restrict__ kb, const uint4* __restrict__ vb,
                                 const int* __restrict__ slot_pos, const float* __restrict__ ks,
                                 const float* __restrict__ vs, int t, int lane) {
  load_tile_k<D>(T, kb, slot_pos, ks, t, lane);
  load_tile_v<D>(T, vb, vs, t, lane);
}

// A tile reload that does nothing (the double-buffered scans load whole tiles themselves).
struct NoLoad {
  template <class T>
  __device__ void operator()(T&) const {}
};

// 8 E4M3 codes (two dwords, element 0 in the low byte) as 8 BF16 values, exactly.
__device__ inline bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, false);
  const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.f, true);
  const auto c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, false);
  const auto d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// scan_tile for an FP8 tile: each K and V operand is converted once and used for every q-block; the raw scores are
// multiplied by their key's scale before the mask, and the softmax weights by their value's scale on the way into
// the P.V product (the running sum takes them unscaled). next_k / next_v: the skewed reload of scan_tile_skewed
// (heads of more than 128 dims), after the scores (K codes, positions, key scales) and after P.V (V codes, value
// scales).
template <int D, int QB, class QS, class LK = NoLoad, class LV = NoLoad>
__device__ inline void scan_tile(KvTile8<D>& T, const QS& qop, const int (&lo)[QB], ScanState<D, QB>& st, int pos0,
                                 LK&& next_k = LK{}, LV&& next_v = LV{}) {
  constexpr int NP = D / 64, NV = D / 32;
  const int kpos[8] = {T.p0.x, T.p0.y, T.p0.z, T.p0.w, T.p1.x, T.p1.y, T.p1.z, T.p1.w};
  const float ks[8] = {T.ks0.x, T.ks0.y, T.ks0.z, T.ks0.w, T.ks1.x, T.ks1.y, T.ks1.z, T.ks1.w};
  const float vs[8] = {T.vs0.x, T.vs0.y, T.vs0.z, T.vs0.w, T.vs1.x, T.vs1.y, T.vs1.z, T.vs1.w};
  f32x4 s[QB][2];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) s[qb][0] = s[qb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      const bf16x8 A0 = fp8x8_to_bf16(T.k[b][c].x, T.k[b][c].y);   // chunk 2 c
      const bf16x8 A1 = fp8x8_to_bf16(T.k[b][c].z, T.k[b][c].w);   // chunk 2 c + 1
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int term = 0; term < 3; ++term) {
          s[qb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, qop.get(qb, 2 * c, term), s[qb][b], 0, 0, 0);
          s[qb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, qop.get(qb, 2 * c + 1, term), s[qb][b], 0, 0, 0);
        }
    }
  next_k(T);   // kpos and ks are copies: the next tile's K half may land in T
  bf16x8 phi[QB], plo[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    float sc[8];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sc[e] = kpos[e] >= lo[qb] && kpos[e] < pos0 ? s[qb][e >> 2][e & 3] * ks[e] : -INFINITY;
      mx = fmaxf(mx, sc[e]);
    }
    mx = xor32_max(xor16_max(mx));
    const float m_new = fmaxf(st.m[qb], mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float corr = exp2_fast(st.m[qb] - m_ref);
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = exp2_fast(sc[e] - m_ref);
      ps += p[e];
    }
    ps = xor32_sum(xor16_sum(ps));
    st.l[qb] = st.l[qb] * corr + ps;
    st.m[qb] = m_new;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pv = p[e] * vs[e];
      const __bf16 h = to_bf16(pv);
      phi[qb][e] = h;
      plo[qb][e] = to_bf16(pv - of_bf16(h));
    }
    if (__ballot(corr != 1.f)) {
#pragma unroll
      for (int dd = 0; dd < D / 16; ++dd) st.acc[qb][dd] *= corr;
    }
  }
#pragma unroll
  for (int dp = 0; dp < NV; ++dp) {
    const bf16x8 A0 = fp8x8_to_bf16(T.v[dp].x, T.v[dp].y);   // block 2 dp
    const bf16x8 A1 = fp8x8_to_bf16(T.v[dp].z, T.v[dp].w);   // block 2 dp + 1
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      f32x4& x0 = st.acc[qb][2 * dp];
      f32x4& x1 = st.acc[qb][2 * dp + 1];
      x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, phi[qb], x0, 0, 0, 0);
      x0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, plo[qb], x0, 0, 0, 0);
      x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, phi[qb], x1, 0, 0, 0);
      x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, plo[qb], x1, 0, 0, 0);
    }
  }
  next_v(T);
}

// LDS of a scan work-group. The q operand in registers: the wave merge, then (raw q rows) the processed q-cols and
// the rows' RoPE cosines and sines. The q operand in LDS: the operand first, then one region that holds the processed
// q-cols and the RoPE table before the scan and the wave merge after it; the merge runs in passes of 128 dims.
template <int D>
constexpr int scan_merge_passes() { return D > 128 ? D / 128 : 1; }
template <int D, int QB, bool RAWQ>
constexpr int scan_qop_floats() { return q_in_lds<D, RAWQ>() ? QB * (D / 32) * 3 * 64 * 4 : 0; }
template <int D, int QB>
constexpr int scan_merge_floats() {
  return kWaves * QB * 2 * 16 + kWaves * QB * (D / 16 / scan_merge_passes<D>()) * 64 * 4;
}
// Row stride of the processed q-cols in LDS: D + 4 floats. The operand build reads 16 q-cols at one dim offset
// per instruction; at a stride of D (a multiple of the bank count) those 16 reads share one bank.
template <int D>
constexpr int sq_stride() { return D + 4; }
template <int D, int QB, bool RAWQ>
constexpr int scan_rawq_floats() { return RAWQ ? QB * 16 * sq_stride<D>() : 0; }
template <int D, int QB, bool RAWQ>
constexpr int scan_sq_offset() {
  return q_in_lds<D, RAWQ>() ? scan_qop_floats<D, QB, RAWQ>() : scan_merge_floats<D, QB>();
}
template <int D, int QB, bool RAWQ>
constexpr int scan_lds_floats() {
  return q_in_lds<D, RAWQ>()
             ? scan_qop_floats<D, QB, RAWQ>() + std::max(scan_merge_floats<D, QB>(), scan_rawq_floats<D, QB, RAWQ>())
             : scan_merge_floats<D, QB>() + scan_rawq_floats<D, QB, RAWQ>();
}

// One scan work-group (KV head, split) of a row block. RAWQ: q arrives as the projection wrote it, and the work-group
// applies the producer's RoPE, justnorm and qscale itself (packs/dory/dory.cpp:482-490) before the scale, once per
// q-col: 16 / QB threads per q-col take d / 2 * QB / 16 consecutive RoPE pairs (i, i + d/2) each with their
// angles' cosines and sines from the position's row of the RoPE table, rotate them, add their squares over those
// lanes, scale, and leave the processed q-col in LDS, from which every lane takes its operand dims.
template <int D, int QB, bool F8, bool RAWQ>
__device__ inline void scan_split(const ScanArgs& a, int bx, float* lds) {
  constexpr int NC = D / 32, ND = D / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int kvh = bx / a.splits, split = bx % a.splits;
  const int blk = a.b0 + int(blockIdx.y), row0 = blk * a.rpb;
  const int qcols = min(a.rpb, a.n_q - row0) * a.group;
  const float* __restrict__ qrows = a.q + size_t(row0) * size_t(a.heads) * D;
  float* __restrict__ acc_out = a.acc + size_t(blk) * a.blk_records * D;
  float* __restrict__ ml_out = a.ml + size_t(blk) * a.blk_records * 2;

  // this split's tiles (at least one: splits <= tiles), dealt to the waves round-robin; the first tile's loads go
  // out before the q operands are built, and every later tile's while the previous one is worked on (an index
  // past the split's end loads its last tile again and is not used)
  const int t_begin = a.tile_lo + int((long long)a.tiles * split / a.splits);
  const int t_end = a.tile_lo + int((long long)a.tiles * (split + 1) / a.splits);
  const int t_last = t_end - 1;
  // per head: slots_pad * D elements of K and of V (16 bytes = 8 BF16 or 16 FP8 per uint4)
  const size_t head_u4 = size_t(a.slots_pad) * size_t(D) / (F8 ? 16 : 8);
  const uint4* kbase = a.ck + size_t(kvh) * head_u4;
  const uint4* vbase = a.cv + size_t(kvh) * head_u4;
  const float* ksb = F8 ? a.kscale + size_t(kvh) * size_t(a.slots_pad) : nullptr;
  const float* vsb = F8 ? a.vscale + size_t(kvh) * size_t(a.slots_pad) : nullptr;
  using Tile = std::conditional_t<F8, KvTile8<D>, KvTile<D>>;
  auto load = [&](Tile& T, int tt) {
    if constexpr (F8)
      load_tile<D>(T, kbase, vbase, a.slot_pos, ksb, vsb, tt, lane);
    else
      load_tile<D>(T, kbase, vbase, a.slot_pos, tt, lane);
  };
  int t = t_begin + wave;
  // heads of 128 dims or more hold one tile, reloaded in a skew (scan_tile_skewed); 64-dim heads alternate two.
  // On 128-dim heads the skew measured 1 % faster per decode step (one- and 8-row steps, 4K and 32K) than two
  // alternating tiles, whose loop the compiler entered with a wait for every outstanding load before the next
  // tile's loads went out.
  constexpr bool SKEW = D >= 128;
  Tile A;
  std::conditional_t<SKEW, char, Tile> B;
  // raw q: the tile's loads go out right after the few q loads, so the q processing waits only for those (loads
  // complete in order); otherwise first
  if constexpr (!RAWQ) load(A, min(t, t_last));

  // q operands: column j of q-block qb is q-col qb * 16 + j = (row, head in the group); times scale * log2(e),
  // three terms. lo: the first stored position the column sees.
  constexpr bool QL = q_in_lds<D, RAWQ>();
  std::conditional_t<QL, QLds<D, QB>, QRegs<D, QB>> qop;
  bf16x8* qlds = reinterpret_cast<bf16x8*>(lds);   // QL: the operand's LDS region
  // QL: each wave builds the chunks c = wave (mod 4) of every q-block into LDS; else every wave all of them
  auto put = [&](int qb, int c, const float (&x)[8]) {
    if constexpr (QL) {
      bf16x8 t0, t1, t2;
      split3(x, t0, t1, t2);
      qlds[((qb * NC + c) * 3 + 0) * 64 + lane] = t0;
      qlds[((qb * NC + c) * 3 + 1) * 64 + lane] = t1;
      qlds[((qb * NC + c) * 3 + 2) * 64 + lane] = t2;
    } else {
      split3(x, qop.q[qb][c][0], qop.q[qb][c][1], qop.q[qb][c][2]);
    }
  };
  constexpr int c_step = QL ? kWaves : 1;
  const int c_first = QL ? wave : 0;
  int lo[QB];
  bool qlive[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qc = qb * 16 + j;
    qlive[qb] = qc < qcols;
    const int qpos = a.pos0 + row0 + (qlive[qb] ? qc / a.group : 0);
    lo[qb] = !qlive[qb] ? INT_MAX : (a.window > 0 ? max(0, qpos - a.window + 1) : 0);
  }
  if constexpr (RAWQ) {
    constexpr int HALF = D / 2;
    constexpr int TPV = 16 / QB;          // threads per q-col
    constexpr int PP = HALF / TPV;        // RoPE pairs per thread
    static_assert(PP % 2 == 0 && TPV * QB * 16 == kWaves * 64, "q-col split");
    constexpr int SQS = sq_stride<D>();
    float* sq = lds + scan_sq_offset<D, QB, RAWQ>();   // processed q-cols [QB * 16][SQS]
    const int v = int(threadIdx.x) / TPV, p0 = (int(threadIdx.x) % TPV) * PP;
    const bool vlive = v < qcols;
    const int vrow = vlive ? v / a.group : 0;
    const int vh = kvh * a.group + (vlive ? v % a.group : 0);
    // every load first: the q-col's pairs, their scales and their angles' (cos, sin) from the position's row
    float x1[PP], x2[PP], s1[PP], s2[PP], cs[PP], sn[PP];
    const float* qp = qrows + (size_t(vrow) * size_t(a.heads) + size_t(vh)) * D;
    const float2* rp = a.rope + (a.plain ? size_t(0) : size_t(a.pos0 + row0 + vrow) * HALF) + p0;
#pragma unroll
    for (int e = 0; e < PP; e += 2) {   // PP consecutive pairs at a multiple of PP: 16-byte loads
      const float4 r = *reinterpret_cast<const float4*>(rp + e);
      cs[e] = r.x, sn[e] = r.y, cs[e + 1] = r.z, sn[e + 1] = r.w;
    }
#pragma unroll
    for (int e = 0; e < PP; e += 2) {   // PP consecutive floats at a multiple of PP: 8-byte loads at least
      const float2 t1 = *reinterpret_cast<const float2*>(qp + p0 + e);
      const float2 t2 = *reinterpret_cast<const float2*>(qp + HALF + p0 + e);
      x1[e] = t1.x, x1[e + 1] = t1.y;
      x2[e] = t2.x, x2[e + 1] = t2.y;
      if (a.qscale) {
        const float* sp = a.qscale + size_t(vh) * D + p0 + e;
        const float2 u1 = *reinterpret_cast<const float2*>(sp);
        const float2 u2 = *reinterpret_cast<const float2*>(sp + HALF);
        s1[e] = u1.x, s1[e + 1] = u1.y;
        s2[e] = u2.x, s2[e + 1] = u2.y;
      } else {
        s1[e] = s1[e + 1] = s2[e] = s2[e + 1] = 1.f;
      }
    }
    load(A, min(t, t_last));
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < PP; ++e) {
      const float o1 = x1[e] * cs[e] - x2[e] * sn[e], o2 = x2[e] * cs[e] + x1[e] * sn[e];
      x1[e] = o1;
      x2[e] = o2;
      ss += o1 * o1 + o2 * o2;
    }
    // the sum over the q-col's TPV consecutive lanes (8 or 16: DPP within rows of 16)
    ss += dpp<kDppXor1>(ss);
    ss += dpp<kDppXor2>(ss);
    ss += dpp<kDppHalfMirror>(ss);
    if constexpr (TPV == 16) ss += dpp<kDppMirror>(ss);
    const float f = a.plain ? 1.f : inv_norm_of(ss);
#pragma unroll
    for (int e = 0; e < PP; e += 2) {
      *reinterpret_cast<float2*>(sq + v * SQS + p0 + e) = make_float2((x1[e] * f) * s1[e], (x1[e + 1] * f) * s1[e + 1]);
      *reinterpret_cast<float2*>(sq + v * SQS + HALF + p0 + e) =
          make_float2((x2[e] * f) * s2[e], (x2[e + 1] * f) * s2[e + 1]);
    }
    __syncthreads();
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int c = c_first; c < NC; c += c_step) {
        const float* sp = sq + (qb * 16 + j) * SQS + 32 * c + 8 * g;
        const float4 u = *reinterpret_cast<const float4*>(sp);
        const float4 w = *reinterpret_cast<const float4*>(sp + 4);
        float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = qlive[qb] ? x[e] * a.scale2 : 0.f;
        put(qb, c, x);
      }
  } else {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qc = qb * 16 + j;
      const int qrow = qlive[qb] ? qc / a.group : 0;
      const float* qp =
          qrows + (size_t(qrow) * size_t(a.heads) + size_t(kvh * a.group + (qlive[qb] ? qc % a.group : 0))) * D;
#pragma unroll
      for (int c = c_first; c < NC; c += c_step) {
        const float4 u = *reinterpret_cast<const float4*>(qp + 32 * c + 8 * g);
        const float4 w = *reinterpret_cast<const float4*>(qp + 32 * c + 8 * g + 4);
        float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = qlive[qb] ? x[e] * a.scale2 : 0.f;
        put(qb, c, x);
      }
    }
  }
  if constexpr (QL) {
    qop.base = qlds;
    qop.lane = lane;
    __syncthreads();   // the operand complete in LDS
  }

  ScanState<D, QB> st;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    st.m[qb] = -INFINITY;
    st.l[qb] = 0.f;
#pragma unroll
    for (int dd = 0; dd < ND; ++dd) st.acc[qb][dd] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (SKEW) {
    (void)B;
    while (t < t_end) {
      const int tn = min(t + kWaves, t_last);
      __asm__ volatile("" ::: "memory");   // keeps the q operand's LDS reads inside the loop
      if constexpr (F8)
        scan_tile<D, QB>(
            A, qop, lo, st, a.pos0, [&](Tile& T) { load_tile_k<D>(T, kbase, a.slot_pos, ksb, tn, lane); },
            [&](Tile& T) { load_tile_v<D>(T, vbase, vsb, tn, lane); });
      else
        scan_tile_skewed<D, QB>(
            A, qop, lo, st, a.pos0, [&](Tile& T) { load_tile_k<D>(T, kbase, a.slot_pos, tn, lane); },
            [&](Tile& T) { load_tile_v<D>(T, vbase, tn, lane); });
      t += kWaves;
    }
  } else {
    while (t < t_end) {
      load(B, min(t + kWaves, t_last));
      if constexpr (QL) __asm__ volatile("" ::: "memory");
      scan_tile<D, QB>(A, qop, lo, st, a.pos0);
      t += kWaves;
      if (t >= t_end) break;
      load(A, min(t + kWaves, t_last));
      if constexpr (QL) __asm__ volatile("" ::: "memory");
      scan_tile<D, QB>(B, qop, lo, st, a.pos0);
      t += kWaves;
    }
  }

  // merge the 4 waves' states in LDS: (max, sum) as [wave][qb][2][16 cols], then accumulators
  // [wave][qb][dd][64 lanes][4], NDP dim blocks at a time (one pass for heads of up to 128 dims)
  constexpr int MP = scan_merge_passes<D>(), NDP = ND / MP;
  float* ml = lds + scan_qop_floats<D, QB, RAWQ>();
  float* accs = ml + kWaves * QB * 2 * 16;   // QL: the region the q-cols were processed in (read before the barrier
                                             // that completed the operand)
#pragma unroll
  for (int pass = 0; pass < MP; ++pass) {
    if (pass > 0) __syncthreads();   // the previous pass's reads are done
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if (g == 0 && pass == 0) {
        ml[((wave * QB + qb) * 2 + 0) * 16 + j] = st.m[qb];
        ml[((wave * QB + qb) * 2 + 1) * 16 + j] = st.l[qb];
      }
#pragma unroll
      for (int dd = 0; dd < NDP; ++dd)
        *reinterpret_cast<f32x4*>(accs + ((size_t(wave * QB + qb) * NDP + dd) * 64 + lane) * 4) =
            st.acc[qb][pass * NDP + dd];
    }
    __syncthreads();
    // wave w finishes q-block w: the partial (max, sum, accumulator[D]) of each live q-col
    for (int qb = wave; qb < QB; qb += kWaves) {
      const int qc = qb * 16 + j;
      float M = -INFINITY;
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[((w * QB + qb) * 2 + 0) * 16 + j]);
      float L = 0.f, f[kWaves];
      for (int w = 0; w < kWaves; ++w) {
        const float mw = ml[((w * QB + qb) * 2 + 0) * 16 + j];
        f[w] = mw == -INFINITY ? 0.f : exp2_fast(mw - M);
        L += f[w] * ml[((w * QB + qb) * 2 + 1) * 16 + j];
      }
      if (qc >= qcols) continue;
      const size_t rec = (size_t(kvh) * size_t(a.splits1) + size_t(split)) * size_t(a.qpad) + size_t(qc);
      if (g == 0 && pass == 0) *reinterpret_cast<float2*>(ml_out + rec * 2) = make_float2(M, L);
      for (int dd = 0; dd < NDP; ++dd) {
        f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < kWaves; ++w)
          s += f[w] * *reinterpret_cast<const f32x4*>(accs + ((size_t(w * QB + qb) * NDP + dd) * 64 + lane) * 4);
        *reinterpret_cast<f32x4*>(acc_out + rec * D + 16 * (pass * NDP + dd) + 4 * g) = s;
      }
    }
  }
}

template <int D, int QB, bool F8>
__global__ void __launch_bounds__(kWaves * 64) attn_scan_kernel(const ScanArgs a) {
  extern __shared__ float lds[];
  scan_split<D, QB, F8, false>(a, int(blockIdx.x), lds);
}

// --------------------------------------------------------------------------------------------------- own keys

// The online-softmax state of one q-col over own keys j0 .. j1 - 1 (kv.cpp:214-243 with this call's FP32 rows),
// computed by one wave. Scores: lane (key slot kk = lane / 8, part p = lane % 8) dots D / 8 dims of q with the same
// dims of key jb + kk, the 8 lanes of a slot add up with three DPP steps, and each slot's score is read out as a
// wave-uniform value. Outputs: lane l holds the OWN_NA<D> dims (l mod OWN_STRIDE<D>) + OWN_STRIDE<D> u (a[u]). q at
// qp, key / value rows at kb + j * stride, vb + j * stride; every load index is clamped into the rows, so none sits
// behind a branch. Scores are in the base-2 domain (scale2 = scale * log2 e).
template <int D>
constexpr int own_na() { return D / 64 > 2 ? D / 64 : 2; }
template <int D>
constexpr int own_stride() { return D / own_na<D>(); }
template <int D>
__device__ inline void own_state(const float* qp, const float* kb, const float* vb, size_t stride, int j0, int j1,
                                 float scale2, float& M, float& L, float (&a)[own_na<D>()]) {
  constexpr int P = D / 8, NA = own_na<D>(), SD = own_stride<D>();
  const int lane = threadIdx.x & 63, slot = lane >> 3, part = lane & 7, l = lane & (SD - 1);
  float q[P];
#pragma unroll
  for (int e = 0; e < P; e += 4) {
    const float4 t = *reinterpret_cast<const float4*>(qp + part * P + e);
    q[e] = t.x, q[e + 1] = t.y, q[e + 2] = t.z, q[e + 3] = t.w;
  }
  for (int jb = j0; jb < j1; jb += 8) {
    const float* kr = kb + size_t(min(jb + slot, j1 - 1)) * stride + part * P;
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < P; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(kr + e);
      dot += q[e] * t.x + q[e + 1] * t.y + q[e + 2] * t.z + q[e + 3] * t.w;
    }
    float vv[8][NA];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const size_t r = size_t(min(jb + u, j1 - 1)) * stride;
#pragma unroll
      for (int n = 0; n < NA; ++n) vv[u][n] = vb[r + l + n * SD];
    }
    dot += dpp<kDppXor1>(dot);
    dot += dpp<kDppXor2>(dot);
    dot += dpp<kDppHalfMirror>(dot);
    const float sc = jb + slot < j1 ? dot * scale2 : -INFINITY;
    float sj[8], bm = -INFINITY;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      sj[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), 8 * u));
      bm = fmaxf(bm, sj[u]);
    }
    const float mn = fmaxf(M, bm);   // finite: the batch holds at least one key
    const float corr = exp2_fast(M - mn);
    L *= corr;
#pragma unroll
    for (int n = 0; n < NA; ++n) a[n] *= corr;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float w = exp2_fast(sj[u] - mn);   // 0 for a slot past j1 (score -inf)
      L += w;
#pragma unroll
      for (int n = 0; n < NA; ++n) a[n] += w * vv[u][n];
    }
    M = mn;
  }
}

template <int D>
__device__ inline void write_partial(float* acc, float* ml, size_t rec, float M, float L,
                                     const float (&a)[own_na<D>()]) {
  const int l = threadIdx.x & 63;
  if (l == 0) *reinterpret_cast<float2*>(ml + rec * 2) = make_float2(M, L);
  if (l < own_stride<D>()) {
#pragma unroll
    for (int n = 0; n < own_na<D>(); ++n) acc[rec * D + l + n * own_stride<D>()] = a[n];
  }
}

// Own keys on the matrix cores (FP32 MFMA 16x16x4), for calls of many rows: one wave per tile of 16 q-cols of a
// row block and chunk of kOwnChunk keys of the range any of its columns sees (from the range's first key), 16 keys
// a step; each chunk leaves its own partial record (own-key record `splits + chunk`), an empty chunk the record of
// no key (max -inf, sum 0), which the merges skip. Chunks put several waves on a SIMD where one wave per column
// tile had every step wait for its loads.
//   S^T (16 keys x 16 q-cols) = K Q^T: at step s lane group g (lane / 16) feeds dim (D / 4) g + s of key / q-col
//   lane % 16, so each lane's K and Q values are D / 4 contiguous floats; lane (g, j) gets S^T[key 4 g + r][col j].
//   O^T (D x 16 q-cols) += V^T P^T: step r sums keys 4 g + r over the lane groups, so P^T comes straight from the
//   scores' registers; lane (g, j) holds O^T[16 t + 4 g + r][col j] in accumulator t.
// The online softmax runs per column over the lane groups (max and sum through two xor shuffles); the partial
// record (M, L, O) goes to the own-key slot (split index `splits`) of the column's block.
struct OwnArgs {
  const float* q;          // [n_own][heads][D]
  const float* k;          // [n_own][kv_heads][D]
  const float* v;
  float* acc;              // partials as ScanArgs
  float* ml;
  size_t blk_records;
  int b0, nblocks, rpb, n_own, heads, kv_heads, group, window, splits, splits1, qpad, tiles;   // tiles per block
  int own;                 // key chunks per column tile
  float scale2;
};

template <int D>
__global__ void __launch_bounds__(256) attn_own_mfma_kernel(const OwnArgs a) {
  constexpr int S = D / 4, T = D / 16;
  const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
  const int w = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
  const int per_blk = a.kv_heads * a.tiles * a.own;
  if (w >= per_blk * a.nblocks) return;   // no barriers below: a spare wave just leaves
  // the last (longest) blocks first; a tile's chunks in consecutive waves (one work-group shares its q loads)
  const int blk = a.b0 + a.nblocks - 1 - w / per_blk, ct = (w % per_blk) / a.own, chunk = w % a.own;
  const int kvh = ct / a.tiles, tile = ct % a.tiles;
  const int row0 = blk * a.rpb, n_rows = min(a.rpb, a.n_own - row0), cols = n_rows * a.group;
  const int qc = tile * 16 + j;
  if (tile * 16 >= cols) return;           // a padding tile of the block
  const bool live = qc < cols;
  const int r = live ? qc / a.group : 0, i = row0 + r;
  const int lo = a.window > 0 ? max(0, i - a.window + 1) : 0;
  // the tile's key range: its rows run from the first column's to the last live column's
  const int i_first = row0 + (tile * 16) / a.group, i_last = row0 + (min(tile * 16 + 15, cols - 1)) / a.group;
  const int k0 = a.window > 0 ? max(0, i_first - a.window + 1) : 0;
  const int kmin = k0 + chunk * kOwnChunk, kmax = min(i_last + 1, kmin + kOwnChunk);   // this chunk's keys

  float qv[S];
  {
    const float* qp = a.q + (size_t(i) * size_t(a.heads) + size_t(kvh * a.group + (live ? qc % a.group : 0))) * D + S * g;
#pragma unroll
    for (int e = 0; e < S; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(qp + e);
      qv[e] = t.x, qv[e + 1] = t.y, qv[e + 2] = t.z, qv[e + 3] = t.w;
    }
  }
  const size_t stride = size_t(a.kv_heads) * D;
  const float* kbase = a.k + size_t(kvh) * D + S * g;
  const float* vbase = a.v + size_t(kvh) * D + j;
  float kn[S], vn[4][T];
  auto load = [&](int kb) {   // key rows past the call's end load its last row (their scores are masked)
    const float* kr = kbase + size_t(min(kb + j, a.n_own - 1)) * stride;
#pragma unroll
    for (int e = 0; e < S; e += 4) {
      const float4 t = *reinterpret_cast<const float4*>(kr + e);
      kn[e] = t.x, kn[e + 1] = t.y, kn[e + 2] = t.z, kn[e + 3] = t.w;
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const float* vr = vbase + size_t(min(kb + 4 * g + rr, a.n_own - 1)) * stride;
#pragma unroll
      for (int t = 0; t < T; ++t) vn[rr][t] = vr[16 * t];
    }
  };
  f32x4 o[T];
#pragma unroll
  for (int t = 0; t < T; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float M = -INFINITY, L = 0.f;
  load(kmin);
  for (int kb = kmin; kb < kmax; kb += 16) {
    float kc[S], vc[4][T];
#pragma unroll
    for (int e = 0; e < S; ++e) kc[e] = kn[e];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int t = 0; t < T; ++t) vc[rr][t] = vn[rr][t];
    load(min(kb + 16, kmax - 1));
    f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < S; ++e) st = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[e], qv[e], st, 0, 0, 0);
    float sc[4], mt = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int key = kb + 4 * g + rr;
      sc[rr] = key >= lo && key <= i ? st[rr] * a.scale2 : -INFINITY;
      mt = fmaxf(mt, sc[rr]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mn = fmaxf(M, mt);
    const float base = mn == -INFINITY ? 0.f : mn;   // no key of the column yet: nothing to rescale
    const float corr = exp2_fast(M - base);
    M = mn;
    float p[4], ps = 0.f;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      p[rr] = exp2_fast(sc[rr] - base);
      ps += p[rr];
    }
    L = L * corr + ps;
#pragma unroll
    for (int t = 0; t < T; ++t) o[t] *= corr;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int t = 0; t < T; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vc[rr][t], p[rr], o[t], 0, 0, 0);
  }
  L += __shfl_xor(L, 16);
  L += __shfl_xor(L, 32);
  if (!live) return;
  const size_t rec = (size_t(kvh) * size_t(a.splits1) + size_t(a.splits + chunk)) * size_t(a.qpad) + size_t(qc);
  float* acc = a.acc + size_t(blk) * a.blk_records * D + rec * D;
  if (g == 0) *reinterpret_cast<float2*>(a.ml + (size_t(blk) * a.blk_records + rec) * 2) = make_float2(M, L);
#pragma unroll
  for (int t = 0; t < T; ++t) *reinterpret_cast<f32x4*>(acc + 16 * t + 4 * g) = o[t];
}

// -------------------------------------------------------------------------------------------------- producer


struct ProduceArgs {
  float* q;                // [m][heads][d], processed in place
  const float* k;          // [m][kv_heads][d]
  const float* v;
  float* kout;             // processed k rows (for a store after the scan), or NULL
  int m, heads, kv_heads, group, window, rpb, splits, splits1, qpad, store;
  long long pos0;
  float scale;
  const float2* rope;      // (cos, sin) of FP32(pos) * inv_freq[i] [pos][d / 2] (launch_rope_table)
  const float* qscale;     // [heads * d] or NULL
  void* ck;                // the cache (BF16, or FP8 codes with the scales below)
  void* cv;
  float* kscale;
  float* vscale;
  int fp8;
  int* slot_pos;
  long long slots;
  int ring, slots_pad;
  float* acc;              // partials of the whole call
  float* ml;
  size_t blk_records;      // records per row block
  int write_q;             // write the processed q rows back in place
  int plain;               // q, k used as they are (the attention call's fused launch; no store, kout or write_q):
                           //   rope is one identity row, read for every position, and no norm
};

// LDS of one producer work-group: row r's processed q heads, the k and v rows it attends to.
template <int D>
constexpr int prod_lds_floats() { return (kProdGroup + 2 * kProdRows) * D; }

// One work-group per (KV head, query row r). It takes RoPE + justnorm of row r's q heads of this KV head (times
// qscale, written back in place) and of the k rows j0 .. r that row r attends to: each work-group recomputes
// those few rows rather than wait for another's. Row r's k and v go to the cache (store set: BF16 as they are
// made, FP8 rows by waves 0 and 1 from LDS once complete, since their scale needs the whole row) and row r's
// processed k to kout (if any); then each q-col of row r gets its own-key partial from one wave. VPW: the rows
// a wave handles (at least ceil((group + r + 1 - j0) / 4)); they are processed without a branch, so their
// reductions interleave.
template <int D, int VPW>
__device__ inline void produce_row(const ProduceArgs& a, int kvh, int r, float* lds) {
  constexpr int HALF = D / 2;
  constexpr int PR = HALF > 64 ? HALF / 64 : 1;   // RoPE pairs (i, i + HALF) per lane: i = l + 64 u
  constexpr int kT = kWaves * 64;
  float* sq = lds;
  float* sk = sq + kProdGroup * D;
  float* sv = sk + kProdRows * D;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool on = lane < HALF;
  const int l = lane & (HALF - 1);
  const int j0 = a.window > 0 ? max(0, r - a.window + 1) : 0;   // the first own key row r sees
  const int nk = r + 1 - j0;                                     // k rows j0 .. r (table rows 0 .. nk - 1)
  const int nv = a.group + nk;                                   // row r's q heads, then those k rows
  const long long slot_r = a.ring ? (a.pos0 + r) % a.slots : a.pos0 + r;

  // every load first, each at an index clamped into its buffer (no load behind a branch): the rows' pairs, their
  // scales, and their angles' (cos, sin) from the RoPE table's row of the row's position (engine/src/kernels.cpp:
  // 203-222: the angle FP32(pos0 + row) * inv_freq[i])
  float x1[VPW][PR], x2[VPW][PR], s1[VPW][PR], s2[VPW][PR];
  float2 cs[VPW][PR];
#pragma unroll
  for (int it = 0; it < VPW; ++it) {
    const int idx = min(wave + it * kWaves, nv - 1);
    const bool is_q = idx < a.group;
    const int h = kvh * a.group + (is_q ? idx : 0);
    const float* p = is_q ? a.q + (size_t(r) * size_t(a.heads) + size_t(h)) * D
                          : a.k + (size_t(j0 + idx - a.group) * size_t(a.kv_heads) + size_t(kvh)) * D;
    const int t = is_q ? nk - 1 : idx - a.group;   // table row: row r for q, row j0 + t for k
    const float2* rp = a.rope + (a.plain ? size_t(0) : size_t(a.pos0 + j0 + t) * HALF);
#pragma unroll
    for (int u = 0; u < PR; ++u) {
      cs[it][u] = rp[l + 64 * u];
      x1[it][u] = p[l + 64 * u];
      x2[it][u] = p[l + 64 * u + HALF];
      s1[it][u] = s2[it][u] = 1.f;
      if (a.qscale && is_q) {
        s1[it][u] = a.qscale[size_t(h) * D + l + 64 * u];
        s2[it][u] = a.qscale[size_t(h) * D + l + 64 * u + HALF];
      }
    }
  }
  constexpr int kVals = (kProdRows * D + kT - 1) / kT;
  float vv[kVals];
#pragma unroll
  for (int u = 0; u < kVals; ++u) {
    const int e = min(tid + u * kT, nk * D - 1);
    vv[u] = a.v[(size_t(j0 + e / D) * size_t(a.kv_heads) + size_t(kvh)) * D + size_t(e % D)];
  }
  // v rows into LDS, row r's into the cache
#pragma unroll
  for (int u = 0; u < kVals; ++u) {
    const int e = tid + u * kT;
    if (e < nk * D) {
      sv[e] = vv[u];
      if (a.store && !a.fp8 && e / D == nk - 1)
        static_cast<uint16_t*>(a.cv)[v_index(kvh, int(slot_r), e % D, a.slots_pad, D)] = f32_to_bf16_bits(vv[u]);
    }
  }
  if (a.store && kvh == 0 && tid == 0) a.slot_pos[slot_r] = int(a.pos0 + r);
  __syncthreads();

#pragma unroll
  for (int it = 0; it < VPW; ++it) {
    const int idx = wave + it * kWaves;
    const bool live = idx < nv;
    const int ic = min(idx, nv - 1);
    const bool is_q = ic < a.group;
    const int t = is_q ? nk - 1 : ic - a.group;   // table row: row r for q, row j0 + t for k
    float o1[PR], o2[PR], ss = 0.f;
#pragma unroll
    for (int u = 0; u < PR; ++u) {
      const float c = cs[it][u].x, s = cs[it][u].y;
      o1[u] = x1[it][u] * c - x2[it][u] * s;
      o2[u] = x2[it][u] * c + x1[it][u] * s;
      ss += o1[u] * o1[u] + o2[u] * o2[u];
    }
    const float f = a.plain ? 1.f : inv_norm_of(wave_sum(on ? ss : 0.f));
#pragma unroll
    for (int u = 0; u < PR; ++u) {
      o1[u] *= f;
      o2[u] *= f;
    }
    if (live && on && is_q) {   // q: times qscale, into LDS (and back in place)
      float* p = a.q + (size_t(r) * size_t(a.heads) + size_t(kvh * a.group + ic)) * D;
#pragma unroll
      for (int u = 0; u < PR; ++u) {
        const int i = lane + 64 * u;
        o1[u] *= s1[it][u];
        o2[u] *= s2[it][u];
        if (a.write_q) {
          p[i] = o1[u];
          p[i + HALF] = o2[u];
        }
        sq[ic * D + i] = o1[u];
        sq[ic * D + i + HALF] = o2[u];
      }
    } else if (live && on) {   // k row j0 + t into LDS; row r's to kout and the cache
#pragma unroll
      for (int u = 0; u < PR; ++u) {
        const int i = lane + 64 * u;
        sk[t * D + i] = o1[u];
        sk[t * D + i + HALF] = o2[u];
        if (t == nk - 1) {
          if (a.kout) {
            float* p = a.kout + (size_t(r) * size_t(a.kv_heads) + size_t(kvh)) * D;
            p[i] = o1[u];
            p[i + HALF] = o2[u];
          }
          if (a.store && !a.fp8) {
            uint16_t* ck = static_cast<uint16_t*>(a.ck);
            ck[k_index(kvh, int(slot_r), i, a.slots_pad, D)] = f32_to_bf16_bits(o1[u]);
            ck[k_index(kvh, int(slot_r), i + HALF, a.slots_pad, D)] = f32_to_bf16_bits(o2[u]);
          }
        }
      }
    }
  }
  __syncthreads();
  if (a.store && a.fp8 && wave < 2) {   // row r's k (wave 0) and v (wave 1), complete in LDS
    const float* src = (wave == 0 ? sk : sv) + (nk - 1) * D;
    float x[D / 64];
#pragma unroll
    for (int u = 0; u < D / 64; ++u) x[u] = src[lane + 64 * u];
    store_fp8_row<D>(x, static_cast<uint8_t*>(wave == 0 ? a.ck : a.cv), wave == 0 ? a.kscale : a.vscale, wave == 1,
                     kvh, int(slot_r), a.slots_pad);
  }

  // own keys: q-col (r, hg) sees keys j0 .. r
  for (int hg = wave; hg < a.group; hg += kWaves) {
    float M = -INFINITY, L = 0.f, acc[own_na<D>()] = {};
    own_state<D>(sq + hg * D, sk, sv, D, 0, nk, a.scale * kLog2e, M, L, acc);
    const int blk = r / a.rpb, qc = (r % a.rpb) * a.group + hg;
    const size_t rec = size_t(blk) * a.blk_records + (size_t(kvh) * size_t(a.splits1) + size_t(a.splits)) * size_t(a.qpad) +
                       size_t(qc);
    write_partial<D>(a.acc, a.ml, rec, M, L, acc);
  }
}

template <int D, int VPW>
__global__ void __launch_bounds__(kWaves * 64) qk_produce_kernel(const ProduceArgs a) {
  __shared__ float lds[prod_lds_floats<D>()];
  produce_row<D, VPW>(a, int(blockIdx.x) % a.kv_heads, int(blockIdx.x) / a.kv_heads, lds);
}

// The decode step's producer and scan in one launch (one row block): work-groups 0 .. kv_heads * splits - 1 scan
// (from the raw q rows, each processing them itself), the last kv_heads * m produce (store, own-key partials;
// q is not written back, since the scan work-groups read it raw). They run concurrently: the scan reads only
// stored positions below pos0 and the store writes only slots that no row sees under their old position nor
// under the new one (the store-first condition), and every slot holds finite values (a new cache is zeroed), so a
// scan that reads a slot while it is rewritten gives it weight 0 either way.
template <int D, int QB, bool F8, int VPW>
__global__ void __launch_bounds__(kWaves * 64) attn_step_kernel(const ScanArgs a, const ProduceArgs pa) {
  extern __shared__ float lds[];
  const int scan_wgs = int(gridDim.x) - pa.kv_heads * pa.m;
  if (int(blockIdx.x) >= scan_wgs) {
    const int pr = int(blockIdx.x) - scan_wgs;
    produce_row<D, VPW>(pa, pr % pa.kv_heads, pr / pa.kv_heads, lds);
    return;
  }
  scan_split<D, QB, F8, true>(a, int(blockIdx.x), lds);
}

// ------------------------------------------------------------------------------------------------------ merge

constexpr int kMergeThreads = 512;

// The online-softmax state (running maximum M in base-2 units, sum L, unnormalised output o) of one q-col for 8 dims
// dd .. dd + 7 over the records rec0 + s * qpad, s = s0, s0 + ds, ... < S1 (kv.cpp:262-285: splits with a zero sum
// are skipped, weights 2^(m_s - max)). The running maximum is updated once per batch of B records, whose loads are
// all in flight together.
template <int D, int B>
__device__ inline void merge8_state(const float* __restrict__ acc, const float* __restrict__ ml, size_t rec0, int qpad,
                                    int s0, int ds, int S1, int dd, float& M, float& L, float (&o)[8]) {
  M = -INFINITY;
  L = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;
  for (int sb = s0; sb < S1; sb += B * ds) {
    float2 w2[B];
    float4 x0[B], x1[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      w2[u] = make_float2(-INFINITY, 0.f);
      x0[u] = x1[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (sb + u * ds < S1) {
        const size_t rec = rec0 + size_t(sb + u * ds) * size_t(qpad);
        w2[u] = *reinterpret_cast<const float2*>(ml + rec * 2);
        x0[u] = *reinterpret_cast<const float4*>(acc + rec * D + dd);
        x1[u] = *reinterpret_cast<const float4*>(acc + rec * D + dd + 4);
      }
    }
    float bm = -INFINITY;
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (w2[u].y != 0.f) bm = fmaxf(bm, w2[u].x);
    const float mn = fmaxf(M, bm);
    if (mn == -INFINITY) continue;
    const float corr = exp2_fast(M - mn);   // M = -inf: 0
    L *= corr;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= corr;
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (w2[u].y != 0.f) {
        const float w = exp2_fast(w2[u].x - mn);
        L += w * w2[u].y;
        o[0] += w * x0[u].x, o[1] += w * x0[u].y, o[2] += w * x0[u].z, o[3] += w * x0[u].w;
        o[4] += w * x1[u].x, o[5] += w * x1[u].y, o[6] += w * x1[u].z, o[7] += w * x1[u].w;
      }
    M = mn;
  }
}

// The merged output over all S1 records (the sum's reciprocal applied last).
template <int D, int B>
__device__ inline void merge8(const float* __restrict__ acc, const float* __restrict__ ml, size_t rec0, int qpad,
                              int S1, int dd, float out[8]) {
  float M, L, o[8];
  merge8_state<D, B>(acc, ml, rec0, qpad, 0, 1, S1, dd, M, L, o);
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = o[e] * inv;
}

struct MergeArgs {
  const float* acc;
  const float* ml;
  int heads, group, rpb, kv_heads, splits1, qpad;
};

// Chunk c (dims 8c .. 8c + 7 of the row's heads * D outputs) of query row `row`.
// The first record of chunk c (dims 8c .. 8c + 7 of the row's heads * D outputs) of query row `row`.
template <int D>
__device__ inline size_t chunk_rec0(const MergeArgs& a, int row, int c) {
  const int h = 8 * c / D;
  const int blk = row / a.rpb, qc = (row % a.rpb) * a.group + h % a.group;
  return ((size_t(blk) * size_t(a.kv_heads) + size_t(h / a.group)) * size_t(a.splits1)) * size_t(a.qpad) + size_t(qc);
}

template <int D, int B>
__device__ inline void merge_chunk(const MergeArgs& a, int row, int c, float out[8]) {
  merge8<D, B>(a.acc, a.ml, chunk_rec0<D>(a, row, c), a.qpad, a.splits1, (8 * c) % D, out);
}

// One work-group per query row: out[row][heads][D].
template <int D>
__global__ void __launch_bounds__(kMergeThreads) attn_merge_kernel(const MergeArgs a, float* __restrict__ out) {
  const int row = blockIdx.x, Q = a.heads * D;
  for (int c = threadIdx.x; c < Q / 8; c += kMergeThreads) {
    float o[8];
    merge_chunk<D, 12>(a, row, c, o);
    float* p = out + size_t(row) * Q + 8 * c;
    *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(o[4], o[5], o[6], o[7]);
  }
}

// One work-group per row of the decode step: merge, a * sigmoid(g * gs), justnorm over the row (dory.cpp:509-515),
// then the FP32 row (out, optional) and the o-projection's operand (optional).
template <int D, int U>
__global__ void __launch_bounds__(kMergeThreads) attn_gate_kernel(const MergeArgs a, const float* __restrict__ g,
                                                                   const float* __restrict__ gs, int vec,
                                                                   float* __restrict__ out, f16x8* __restrict__ xop,
                                                                   float* __restrict__ xinv, size_t ostride) {
  __shared__ float red[2 * kMergeThreads / 64];
  const int row = blockIdx.x, Q = a.heads * D;
  float gv[U][8], sv[U][8], t[U][8];
  load_row<kMergeThreads, U>(g + size_t(row) * Q, Q, vec, gv);
  load_row<kMergeThreads, U>(gs, Q, vec, sv);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = int(threadIdx.x) + u * kMergeThreads;
    if (8 * c < Q) {
      merge_chunk<D, (U == 1 ? 12 : 16 / (2 * U))>(a, row, c, t[u]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) t[u][e] = 0.f;
    }
  }
  float s = 0.f, mx = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      t[u][e] = t[u][e] * (1.f / (1.f + expf(-gv[u][e] * sv[u][e])));
      s += t[u][e] * t[u][e];
      mx = fmaxf(mx, fabsf(t[u][e]));
    }
  // the largest magnitude rides with the sum: max |t f| = fl(max |t| * f) for f > 0
  block_sum_max<kMergeThreads>(s, mx, red);
  const float f = inv_norm_of(s);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) t[u][e] *= f;
  if (out) store_row<kMergeThreads, U>(out + size_t(row) * Q, Q, vec, t);
  if (xop) emit_operand_mx<kMergeThreads, U>(t, Q, row, xop, xinv, ostride, mx * f);
}

// The one-token step's gate with its norm left to the o-projection: W waves per head. Lane l of wave w = (part p,
// chunk c) with CH = D / 8 chunks of 8 dims, P = 64 / CH parts per wave and p = w P + l / CH: part p merges the
// head's records s = p, p + W P, ... (up to 8 of them per batch, all loads in flight together; the host takes W so
// that one batch holds them all where it can, since every further batch is one more round trip of dependent loads:
// 65 records per column, the 32K global layers of an FP8 cache, took three on one wave). Waves 1 .. W - 1 hand
// their lanes' states to wave 0 through LDS, which takes them in wave order; the parts' states are then combined
// across lanes (exchanges of lanes l ^ CH, l ^ 2 CH, ...): the same order every call. Part 0 applies
// a * sigmoid(g * gs) (dory.cpp:509-512), writes the gated head to y and its sum of squares to rec[head], from which
// the o-projection's operand takes the justnorm (dory.cpp:513-515). Without GATE the same merge is the attention
// call's (kv.cpp:262-285) for a call of one row block: head blockIdx.x of row blockIdx.y, merged, into y
// [rows][heads * D].
template <int CH>
__device__ inline float xor_parts_max(float v) {
  if constexpr (CH <= 8) v = fmaxf(v, __shfl_xor(v, 8));
  if constexpr (CH <= 16) v = xor16_max(v);
  return xor32_max(v);
}
template <int CH>
__device__ inline float xor_parts_sum(float v) {
  if constexpr (CH <= 8) v += __shfl_xor(v, 8);
  if constexpr (CH <= 16) v = xor16_sum(v);
  return xor32_sum(v);
}

template <int D, int W, bool GATE>
__device__ inline void merge_heads(const MergeArgs& a, const float* __restrict__ g, const float* __restrict__ gs,
                                   float* __restrict__ y, float* __restrict__ rec) {
  constexpr int CH = D / 8, P = 64 / CH;
  static_assert(CH >= 8 && CH <= 32, "8 to 32 chunks per head");
  __shared__ float hand[W > 1 ? (W - 1) * 10 * 64 : 1];   // waves 1 .. W - 1: [wave][M, L, o[8]][lane]
  const int h = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = GATE ? 0 : int(blockIdx.y);
  const int c = h * CH + lane % CH, p = wave * P + lane / CH;
  // the gate's inputs first (every wave: no load behind a branch; wave 0 uses them)
  float4 g0, g1, s0, s1;
  if constexpr (GATE) {
    g0 = *reinterpret_cast<const float4*>(g + 8 * c), g1 = *reinterpret_cast<const float4*>(g + 8 * c + 4);
    s0 = *reinterpret_cast<const float4*>(gs + 8 * c), s1 = *reinterpret_cast<const float4*>(gs + 8 * c + 4);
  }
  float M, L, o[8];
  merge8_state<D, 8>(a.acc, a.ml, chunk_rec0<D>(a, row, c), a.qpad, p, W * P, a.splits1, (8 * c) % D, M, L, o);
  if constexpr (W > 1) {
    if (wave > 0) {
      float* hp = hand + (wave - 1) * 10 * 64 + lane;
      hp[0] = M;
      hp[64] = L;
#pragma unroll
      for (int e = 0; e < 8; ++e) hp[(2 + e) * 64] = o[e];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < W - 1; ++w) {
      const float* hp = hand + w * 10 * 64 + lane;
      const float M2 = hp[0];
      const float mn = fmaxf(M, M2);
      if (mn == -INFINITY) continue;
      const float f1 = exp2_fast(M - mn), f2 = exp2_fast(M2 - mn);   // -inf: 0
      L = L * f1 + hp[64] * f2;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = o[e] * f1 + hp[(2 + e) * 64] * f2;
      M = mn;
    }
  }
  const float Mh = xor_parts_max<CH>(M);
  const float f = M == -INFINITY ? 0.f : exp2_fast(M - Mh);
  const float Lh = xor_parts_sum<CH>(L * f);
  const float inv = Lh > 0.f ? 1.f / Lh : 0.f;
  float t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = xor_parts_sum<CH>(o[e] * f) * inv;
  if constexpr (!GATE) {
    float* yr = y + size_t(row) * size_t(gridDim.x) * D;
    if (p == 0) {
      *reinterpret_cast<float4*>(yr + 8 * c) = make_float4(t[0], t[1], t[2], t[3]);
      *reinterpret_cast<float4*>(yr + 8 * c + 4) = make_float4(t[4], t[5], t[6], t[7]);
    }
    return;
  } else {
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      t[e] *= 1.f / (1.f + expf(-gv[e] * sv[e]));
      ss += t[e] * t[e];
    }
    if (p == 0) {
      *reinterpret_cast<float4*>(y + 8 * c) = make_float4(t[0], t[1], t[2], t[3]);
      *reinterpret_cast<float4*>(y + 8 * c + 4) = make_float4(t[4], t[5], t[6], t[7]);
    }
    ss = wave_sum(p == 0 ? ss : 0.f);
    if (lane == 0) rec[h] = ss;
  }
}

template <int D, int W>
__global__ void __launch_bounds__(64 * W) attn_gate_heads_kernel(const MergeArgs a, const float* __restrict__ g,
                                                                 const float* __restrict__ gs, float* __restrict__ y,
                                                                 float* __restrict__ rec) {
  merge_heads<D, W, true>(a, g, gs, y, rec);
}

template <int D, int W>
__global__ void __launch_bounds__(64 * W) attn_merge_heads_kernel(const MergeArgs a, float* __restrict__ out) {
  merge_heads<D, W, false>(a, nullptr, nullptr, out, nullptr);
}

// ------------------------------------------------------------------------------------------------------- plan

AttnPlan attn_plan(const DevKv& c, int n_q, int heads, long long pos0, int window) {
  XTG_CHECK(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "attention: head_dim %d (64, 128 or 256)",
            c.head_dim);
  XTG_CHECK(heads % c.kv_heads == 0, "attention: %d heads over %d KV heads", heads, c.kv_heads);
  const int group = heads / c.kv_heads;
  XTG_CHECK(group <= 8, "attention: %d query heads per KV head (at most 8)", group);
  XTG_CHECK(n_q >= 1, "attention: %d query rows", n_q);
  XTG_CHECK(pos0 >= 0 && pos0 + n_q < (1LL << 31), "attention: positions %lld + %d beyond the 32-bit slot positions",
            pos0, n_q);
  AttnPlan p;
  p.group = group;
  p.kv_heads = c.kv_heads;
  p.d = c.head_dim;
  p.rpb = std::max(1, 32 / group);
  p.blocks = (n_q + p.rpb - 1) / p.rpb;
  p.qpad = (std::min(n_q, p.rpb) * group + 15) / 16 * 16;
  if (c.ring) {   // any slot may hold a visible position: scan the whole ring
    p.tile_lo = 0;
    p.tiles = c.slots_pad / kTile;
  } else {        // positions lo(pos0) .. pos0 - 1 live in slots of the same number
    long long lo = window > 0 ? std::max<long long>(0, pos0 - window + 1) : 0;   // row 0 sees the earliest key
    lo = std::max<long long>(0, std::min<long long>(lo, pos0));
    const long long hi = std::min<long long>(pos0, c.slots);
    p.tile_lo = int(lo / kTile);
    p.tiles = hi > lo ? int((hi + kTile - 1) / kTile - lo / kTile) : 0;
  }
  // about 192 work-groups over the KV heads and row blocks, at least two tiles per wave on a cache by position
  // and one on a ring, at most one split per tile. Measured on the 4B-shaped decode step: every split adds a
  // partial record that the gate merges; with the gate's merge in one round of loads, 192 work-groups (24 splits on
  // the global layers) take 1.6 % off the one-token step at 32K and 0.7 % at 8K against 128 (the 8-row step: 0.6 %
  // faster at 32K, 0.4 % slower at 8K), 256 and 384 are slower; one tile per wave on the 1088-slot rings (9 splits
  // instead of 5) takes 1-1.3 % off the 8-row step, while on the global layers it doubles the partials at 4K and
  // costs 2 %. A one-row scan of an E4M3 cache by position has half the bytes per tile for the same conversion
  // work: at 192 work-groups (under one wave per SIMD) its waves issued VALU for 39 % of their cycles and waited for
  // 8 %, and 512 work-groups take 1.5 % off the one-token step at 32K (1.099 -> 1.082 ms, with the gate's merge on
  // more waves; 0.2 % at 8K; 768 and 1024: 1.109 and 1.105 ms), while at 8 rows they cost 4 %.
  // (XTG_ATTN_SPLITS=n fixes the count, for experiments)
  if (p.tiles > 0) {
    const int wgs = c.fp8 && !c.ring && n_q == 1 ? 512 : 192;
    const int want = std::max(1, wgs / (c.kv_heads * p.blocks));   // about wgs work-groups over all blocks
    const int mt = c.ring ? 1 : 2;
    p.splits = std::max(1, std::min(want, (p.tiles + mt * kWaves - 1) / (mt * kWaves)));
    if (const char* env = std::getenv("XTG_ATTN_SPLITS")) p.splits = std::max(1, std::atoi(env));
    p.splits = std::min(p.splits, p.tiles);
  } else {
    p.splits = 0;
  }
  // own keys: a column tile's key range is at most the call's rows, or with a window the window and the block's
  // other rows; the matrix-core own-key kernel takes it in chunks of kOwnChunk keys, a wave each (the producer of a
  // call of up to kProdRows rows writes the one record itself)
  const int own_range = window > 0 ? int(std::min<long long>(n_q, (long long)window + p.rpb - 1)) : n_q;
  p.own = std::max(1, (own_range + kOwnChunk - 1) / kOwnChunk);
  return p;
}

// ------------------------------------------------------------------------------------------ fixed scratch

// The attention call that allocates nothing keeps its split partials here: one array per device, of
// kAttnScratchBytes, shared by every such call on that device (each call writes every partial it reads). Host code
// never passes the array's name to a kernel: in host code it is a stand-in, not a device address. The address each
// device holds it at comes from hipGetSymbolAddress, looked up once per device with that device current.
static __device__ __align__(256) float scratch[kAttnScratchBytes / sizeof(float)];

void* attn_scratch_ptr(int device) {
  static std::mutex mu;
  static std::vector<void*> ptrs;   // per device
  std::lock_guard<std::mutex> lock(mu);
  XTG_CHECK(device >= 0, "attention scratch: device %d", device);
  if (size_t(device) >= ptrs.size()) ptrs.resize(size_t(device) + 1, nullptr);
  if (!ptrs[size_t(device)]) {
    int cur = -1;
    HIP_CHECK(hipGetDevice(&cur));
    XTG_CHECK(cur == device, "attention scratch: device %d is not the current device (%d is)", device, cur);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    XTG_CHECK(e == hipSuccess && p != nullptr, "attention scratch: hipGetSymbolAddress failed on device %d: %s",
              device, hipGetErrorString(e));
    ptrs[size_t(device)] = p;
  }
  return ptrs[size_t(device)];
}

namespace {
std::mutex scratch_mu;
std::vector<const void*> scratch_owner;   // per device: the backend holding the array, or NULL
}  // namespace

bool attn_scratch_claim(int device, const void* owner) {
  std::lock_guard<std::mutex> lock(scratch_mu);
  XTG_CHECK(device >= 0 && owner, "attention scratch: device %d", device);
  if (size_t(device) >= scratch_owner.size()) scratch_owner.resize(size_t(device) + 1, nullptr);
  const void*& o = scratch_owner[size_t(device)];
  if (o && o != owner) return false;
  o = owner;
  return true;
}

void attn_scratch_let_go(int device, const void* owner) {
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (device >= 0 && size_t(device) < scratch_owner.size() && scratch_owner[size_t(device)] == owner)
    scratch_owner[size_t(device)] = nullptr;
}

// ------------------------------------------------------------------------------------------------- launchers

// The RoPE rows of positions 0 .. n_pos - 1: (cos, sin) of the angle FP32(pos) * inv_freq[i] (engine/src/
// kernels.cpp:203-222), [pos][d / 2], the same expression the row kernels evaluate, so a table entry is the value
// they compute for that position.
__global__ void __launch_bounds__(256) rope_table_kernel(const float* __restrict__ inv_freq, int half, long long n_pos,
                                                         float2* __restrict__ out) {
  const long long n = n_pos * half;
  for (long long e = (long long)blockIdx.x * 256 + threadIdx.x; e < n; e += (long long)gridDim.x * 256) {
    const float ang = float(e / half) * inv_freq[e % half];
    out[e] = make_float2(cosf(ang), sinf(ang));
  }
}

std::string launch_rope_table(const float* inv_freq, int d, long long n_pos, float2* out, hipStream_t stream) {
  XTG_CHECK(d % 2 == 0 && d > 0 && n_pos > 0, "rope table: head_dim %d, %lld positions", d, n_pos);
  const long long n = n_pos * (d / 2);
  const unsigned blocks = unsigned(std::min<long long>((n + 255) / 256, 65536));
  hipLaunchKernelGGL(rope_table_kernel, dim3(blocks), dim3(256), 0, stream, inv_freq, d / 2, n_pos, out);
  HIP_CHECK(hipGetLastError());
  return "rope_table_kernel";
}

// The wave merge of a scan needs more than the default 64 KiB of LDS for 128-dim heads and two q-blocks, as does a
// wide GEMV on raw rows: raise the kernel's limit once.
void allow_lds(const void* fn, size_t lds) {
  if (lds <= 65536) return;
  static thread_local const void* raised[128] = {};
  for (const void* f : raised)
    if (f == fn) return;
  HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  for (const void*& f : raised)
    if (!f) {
      f = fn;
      return;
    }
}

namespace {

using ScanFn = void (*)(const ScanArgs);
ScanFn scan_fn(int d, int qb, bool f8) {
#define XTG_CASE(D, Q, F) \
  if (d == D && qb == Q && f8 == F) return attn_scan_kernel<D, Q, F>;
  XTG_CASE(64, 1, false) XTG_CASE(64, 2, false) XTG_CASE(128, 1, false) XTG_CASE(128, 2, false)
  XTG_CASE(64, 1, true) XTG_CASE(64, 2, true) XTG_CASE(128, 1, true) XTG_CASE(128, 2, true)
  XTG_CASE(256, 1, false) XTG_CASE(256, 2, false) XTG_CASE(256, 1, true) XTG_CASE(256, 2, true)
#undef XTG_CASE
  return nullptr;
}

// LDS bytes of a scan launch (raw q rows: the fused decode step's)
size_t scan_lds_bytes(int d, int qb, bool rawq) {
#define XTG_LDS(D, Q)                                                                             \
  if (d == D && qb == Q)                                                                          \
    return size_t(rawq ? scan_lds_floats<D, Q, true>() : scan_lds_floats<D, Q, false>()) * sizeof(float);
  XTG_LDS(64, 1) XTG_LDS(64, 2) XTG_LDS(128, 1) XTG_LDS(128, 2) XTG_LDS(256, 1) XTG_LDS(256, 2)
#undef XTG_LDS
  fail("attention: no scan for head_dim %d and %d column blocks", d, qb);
}


size_t blk_records(const AttnPlan& p) { return size_t(p.kv_heads) * size_t(p.splits + p.own) * size_t(p.qpad); }

MergeArgs merge_args(const AttnPlan& p, int heads, const float* part) {
  MergeArgs a;
  a.acc = part;
  a.ml = part + p.records() * size_t(p.d);
  a.heads = heads;
  a.group = p.group;
  a.rpb = p.rpb;
  a.kv_heads = p.kv_heads;
  a.splits1 = p.splits + p.own;
  a.qpad = p.qpad;
  return a;
}

int block_rows(const AttnPlan& p, int n_q, int b) {
  XTG_CHECK(b >= 0 && b < p.blocks, "attention: block %d of %d", b, p.blocks);
  return std::min(p.rpb, n_q - b * p.rpb);
}

ScanArgs scan_args(const DevKv& c, const AttnPlan& p, int b0, const float* q, int n_q, int heads, long long pos0,
                   int window, float scale, float* part) {
  ScanArgs a{};
  a.q = q;
  a.ck = reinterpret_cast<const uint4*>(c.k);
  a.cv = reinterpret_cast<const uint4*>(c.v);
  a.slot_pos = c.slot_pos;
  a.kscale = c.kscale;
  a.vscale = c.vscale;
  a.acc = part;
  a.ml = part + p.records() * size_t(p.d);
  a.blk_records = blk_records(p);
  a.b0 = b0;
  a.rpb = p.rpb;
  a.n_q = n_q;
  a.heads = heads;
  a.group = p.group;
  a.window = window;
  a.splits = p.splits;
  a.splits1 = p.splits + p.own;
  a.qpad = p.qpad;
  a.slots_pad = c.slots_pad;
  a.tile_lo = p.tile_lo;
  a.tiles = p.tiles;
  a.pos0 = int(pos0);
  a.scale2 = scale * kLog2e;
  return a;
}

ProduceArgs produce_args(const DevKv& c, const AttnPlan& p, float* q, const float* k, const float* v, float* kout,
                         int m, int heads, long long pos0, int window, float scale, const float2* rope,
                         const float* qscale, bool store, float* part) {
  XTG_CHECK(m >= 1 && m <= kProdRows, "producer: %d rows (1..%d)", m, kProdRows);
  XTG_CHECK(p.group <= kProdGroup, "producer: %d query heads per KV head", p.group);
  XTG_CHECK(!store || !c.ring || c.slots >= m, "producer: %d rows into a %lld-slot ring", m, c.slots);
  XTG_CHECK(p.own == 1, "producer: %d own-key records (one)", p.own);
  ProduceArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.kout = kout;
  a.m = m;
  a.heads = heads;
  a.kv_heads = c.kv_heads;
  a.group = p.group;
  a.window = window;
  a.rpb = p.rpb;
  a.splits = p.splits;
  a.splits1 = p.splits + p.own;
  a.qpad = p.qpad;
  a.store = store ? 1 : 0;
  a.pos0 = pos0;
  a.scale = scale;
  a.rope = rope;
  a.qscale = qscale;
  a.ck = c.k;
  a.cv = c.v;
  a.kscale = c.kscale;
  a.vscale = c.vscale;
  a.fp8 = c.fp8 ? 1 : 0;
  a.slot_pos = c.slot_pos;
  a.slots = c.slots;
  a.ring = c.ring ? 1 : 0;
  a.slots_pad = c.slots_pad;
  a.acc = part;
  a.ml = part + p.records() * size_t(p.d);
  a.blk_records = blk_records(p);
  a.write_q = 1;
  return a;
}

// The producer's rows per wave: row r's q heads and the own k rows it sees (at most min(m, window)), over 4 waves.
int produce_vpw(const AttnPlan& p, int m, int window) {
  const int keys = window > 0 ? std::min(m, window) : m;
  const int need = (p.group + keys + kWaves - 1) / kWaves;
  XTG_CHECK(need <= 4, "producer: %d rows per wave", need);
  return need <= 2 ? 2 : 4;
}

}  // namespace

std::string launch_attn_scan(const DevKv& c, const AttnPlan& p, int b0, int nblocks, const float* q, int n_q,
                             int heads, long long pos0, int window, float scale, float* part, hipStream_t stream) {
  XTG_CHECK(p.splits >= 1 && p.splits <= p.tiles, "attention: %d splits over %d tiles", p.splits, p.tiles);
  XTG_CHECK(nblocks >= 1 && b0 + nblocks <= p.blocks, "attention: blocks %d .. %d of %d", b0, b0 + nblocks, p.blocks);
  const int nr = block_rows(p, n_q, b0);   // the widest block of the launch
  const ScanArgs a = scan_args(c, p, b0, q, n_q, heads, pos0, window, scale, part);
  const int qb = (nr * p.group + 15) / 16;
  ScanFn fn = scan_fn(c.head_dim, qb, c.fp8);
  XTG_CHECK(fn != nullptr, "attention: no kernel for head_dim %d and %d column blocks", c.head_dim, qb);
  const size_t lds = scan_lds_bytes(c.head_dim, qb, false);
  allow_lds(reinterpret_cast<const void*>(fn), lds);
  hipLaunchKernelGGL(fn, dim3(unsigned(c.kv_heads * p.splits), unsigned(nblocks)), dim3(kWaves * 64), lds, stream, a);
  HIP_CHECK(hipGetLastError());
  return strf("attn_scan_kernel<%d, %d, %s>", c.head_dim, qb, c.fp8 ? "true" : "false");
}

std::string launch_attn_own(const AttnPlan& p, int b0, int nblocks, const float* q, const float* k, const float* v,
                            int n_q, int heads, int window, float scale, float* part, hipStream_t stream) {
  XTG_CHECK(nblocks >= 1 && b0 + nblocks <= p.blocks, "attention: blocks %d .. %d of %d", b0, b0 + nblocks, p.blocks);
  XTG_CHECK(p.qpad % 16 == 0, "attention: %d padded q-cols", p.qpad);
  OwnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.acc = part;
  a.ml = part + p.records() * size_t(p.d);
  a.blk_records = blk_records(p);
  a.b0 = b0;
  a.nblocks = nblocks;
  a.rpb = p.rpb;
  a.n_own = n_q;
  a.heads = heads;
  a.kv_heads = p.kv_heads;
  a.group = p.group;
  a.window = window;
  a.splits = p.splits;
  a.splits1 = p.splits + p.own;
  a.qpad = p.qpad;
  a.tiles = p.qpad / 16;
  a.own = p.own;
  a.scale2 = scale * kLog2e;
  const long long waves = (long long)p.kv_heads * a.tiles * p.own * nblocks;
  const dim3 grid{unsigned((waves + 3) / 4)}, block{256};
  if (p.d == 64)
    hipLaunchKernelGGL(attn_own_mfma_kernel<64>, grid, block, 0, stream, a);
  else if (p.d == 128)
    hipLaunchKernelGGL(attn_own_mfma_kernel<128>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(attn_own_mfma_kernel<256>, grid, block, 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return strf("attn_own_mfma_kernel<%d>", p.d);
}

std::string launch_attn_merge(const AttnPlan& p, int n_q, int heads, const float* part, float* out,
                              hipStream_t stream) {
  const MergeArgs a = merge_args(p, heads, part);
  if (p.d == 64)
    hipLaunchKernelGGL(attn_merge_kernel<64>, dim3(unsigned(n_q)), dim3(kMergeThreads), 0, stream, a, out);
  else if (p.d == 128)
    hipLaunchKernelGGL(attn_merge_kernel<128>, dim3(unsigned(n_q)), dim3(kMergeThreads), 0, stream, a, out);
  else
    hipLaunchKernelGGL(attn_merge_kernel<256>, dim3(unsigned(n_q)), dim3(kMergeThreads), 0, stream, a, out);
  HIP_CHECK(hipGetLastError());
  return strf("attn_merge_kernel<%d>", p.d);
}

std::string launch_qk_produce(const DevKv& c, const AttnPlan& p, float* q, const float* k, const float* v, float* kout,
                              int m, int heads, long long pos0, int window, float scale, const float2* rope,
                              const float* qscale, bool store, float* part, hipStream_t stream) {
  XTG_CHECK(rope, "producer: no RoPE table");
  const ProduceArgs a = produce_args(c, p, q, k, v, kout, m, heads, pos0, window, scale, rope, qscale, store, part);
  const int vpw = produce_vpw(p, m, window);
  const dim3 grid{unsigned(c.kv_heads * m)}, block{unsigned(kWaves * 64)};
#define XTG_PROD(D, V) \
  if (c.head_dim == D && vpw == V) hipLaunchKernelGGL((qk_produce_kernel<D, V>), grid, block, 0, stream, a);
  XTG_PROD(64, 2) XTG_PROD(64, 4) XTG_PROD(128, 2) XTG_PROD(128, 4) XTG_PROD(256, 2) XTG_PROD(256, 4)
#undef XTG_PROD
  XTG_CHECK(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "producer: head_dim %d", c.head_dim);
  HIP_CHECK(hipGetLastError());
  return strf("qk_produce_kernel<%d, %d>", c.head_dim, vpw);
}

bool attn_step_fuses(const AttnPlan& p, int m) {
  return p.blocks == 1 && p.splits >= 1 && m <= kProdRows && (m * p.group + 15) / 16 <= 2;
}

std::string launch_attn_step(const DevKv& c, const AttnPlan& p, float* q, const float* k, const float* v,
                             float* kout, int m, int heads, long long pos0, int window, float scale,
                             const float2* rope, const float* qscale, bool store, float* part,
                             hipStream_t stream, bool plain) {
  XTG_CHECK(rope, "attention step: no RoPE table");
  XTG_CHECK(!plain || (!store && !kout && !qscale), "attention step: q and k as they are take no store, kout or qscale");
  XTG_CHECK(attn_step_fuses(p, m), "attention step: %d rows in %d blocks, %d splits: no fused launch", m, p.blocks,
            p.splits);
  XTG_CHECK(p.splits <= p.tiles, "attention: %d splits over %d tiles", p.splits, p.tiles);
  XTG_CHECK(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "attention step: head_dim %d", c.head_dim);
  XTG_CHECK(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(qscale) % 16 == 0,
            "attention step: q and qscale must be 16-byte aligned");
  ScanArgs a = scan_args(c, p, 0, q, m, heads, pos0, window, scale, part);
  a.rope = rope;
  a.qscale = qscale;
  ProduceArgs pa = produce_args(c, p, q, k, v, kout, m, heads, pos0, window, scale, rope, qscale, store, part);
  pa.write_q = 0;   // the scan work-groups read q raw while the producers run
  a.plain = pa.plain = plain ? 1 : 0;
  const int vpw = produce_vpw(p, m, window);
  const int qb = (m * p.group + 15) / 16;
  const dim3 grid{unsigned(c.kv_heads * p.splits + c.kv_heads * m)}, block{unsigned(kWaves * 64)};
  bool done = false;
#define XTG_STEP(D, Q, F, V)                                                                                   \
  if (!done && c.head_dim == D && qb == Q && c.fp8 == F && vpw == V) {                                         \
    auto fn = attn_step_kernel<D, Q, F, V>;                                                                    \
    const size_t lds = std::max(scan_lds_bytes(D, Q, true), size_t(prod_lds_floats<D>()) * sizeof(float));     \
    allow_lds(reinterpret_cast<const void*>(fn), lds);                                                         \
    hipLaunchKernelGGL(fn, grid, block, lds, stream, a, pa);                                                   \
    done = true;                                                                                               \
  }
#define XTG_STEP_D(D) \
  XTG_STEP(D, 1, false, 2) XTG_STEP(D, 1, false, 4) XTG_STEP(D, 2, false, 2) XTG_STEP(D, 2, false, 4) \
  XTG_STEP(D, 1, true, 2) XTG_STEP(D, 1, true, 4) XTG_STEP(D, 2, true, 2) XTG_STEP(D, 2, true, 4)
  XTG_STEP_D(64) XTG_STEP_D(128) XTG_STEP_D(256)
#undef XTG_STEP_D
#undef XTG_STEP
  XTG_CHECK(done, "attention step: no kernel for head_dim %d, %d column blocks, %d rows per wave", c.head_dim, qb,
            vpw);
  HIP_CHECK(hipGetLastError());
  return strf("attn_step_kernel<%d, %d, %s, %d>", c.head_dim, qb, c.fp8 ? "true" : "false", vpw);
}

std::string launch_attn_gate(const AttnPlan& p, int m, int heads, const float* part, const float* g, const float* gs,
                             float* out, void* op, hipStream_t stream) {
  const MergeArgs a = merge_args(p, heads, part);
  const int Q = heads * p.d;
  f16x8* xop = nullptr;
  float* xinv = nullptr;
  if (op) {
    XTG_CHECK(m <= kMaxOperandRows, "attention gate: %d rows for an operand", m);
    xop = static_cast<f16x8*>(op);
    xinv = reinterpret_cast<float*>(static_cast<char*>(op) + xop_bytes(Q));
  }
  auto al = [](const void* x) { return !x || reinterpret_cast<uintptr_t>(x) % 16 == 0; };
  const int vec = al(g) && al(gs) && al(out) ? 1 : 0;
  const int chunks = Q / 8;
  const dim3 grid{unsigned(m)}, block{unsigned(kMergeThreads)};
  int u = 0;
#define XTG_GATE(D, U)                                                                                      \
  if (p.d == D && chunks <= U * kMergeThreads && !u) {                                                      \
    hipLaunchKernelGGL((attn_gate_kernel<D, U>), grid, block, 0, stream, a, g, gs, vec, out, xop, xinv,    \
                       op_group_bytes(Q));                                                               \
    u = U;                                                                                                  \
  }
  XTG_GATE(64, 1) XTG_GATE(64, 2) XTG_GATE(64, 4) XTG_GATE(128, 1) XTG_GATE(128, 2) XTG_GATE(128, 4)
  XTG_GATE(256, 1) XTG_GATE(256, 2) XTG_GATE(256, 4)
#undef XTG_GATE
  XTG_CHECK(u != 0, "attention gate: %d heads of %d", heads, p.d);
  HIP_CHECK(hipGetLastError());
  return strf("attn_gate_kernel<%d, %d>", p.d, u);
}

// waves per head of a merge by heads: enough parts (64 / (d / 8) per wave) for a column's records to fit one batch of
// 8 each, at most 4
int merge_heads_waves(const AttnPlan& p, int records) {
  const int parts = (records + 7) / 8, per_wave = 64 / (p.d / 8);
  const int need = (parts + per_wave - 1) / per_wave;
  return need <= 1 ? 1 : need <= 2 ? 2 : 4;
}

std::string launch_attn_gate_heads(const AttnPlan& p, int heads, const float* part, const float* g, const float* gs,
                                   float* y, float* rec, hipStream_t stream) {
  XTG_CHECK(p.blocks == 1, "attention gate by heads: one query row");
  auto al = [](const void* x) { return reinterpret_cast<uintptr_t>(x) % 16 == 0; };
  XTG_CHECK(g && gs && y && rec && al(g) && al(gs) && al(y), "attention gate by heads: 16-byte aligned rows");
  const MergeArgs a = merge_args(p, heads, part);
  XTG_CHECK(p.d == 64 || p.d == 128 || p.d == 256, "attention gate by heads: head_dim %d", p.d);
  const int w = merge_heads_waves(p, a.splits1);
  const dim3 grid{unsigned(heads)}, block{unsigned(64 * w)};
#define XTG_GATE_HEADS(D, W)                                                                                  \
  if (p.d == D && w == W)                                                                                     \
    hipLaunchKernelGGL((attn_gate_heads_kernel<D, W>), grid, block, 0, stream, a, g, gs, y, rec);
  XTG_GATE_HEADS(64, 1) XTG_GATE_HEADS(64, 2) XTG_GATE_HEADS(64, 4)
  XTG_GATE_HEADS(128, 1) XTG_GATE_HEADS(128, 2) XTG_GATE_HEADS(128, 4)
  XTG_GATE_HEADS(256, 1) XTG_GATE_HEADS(256, 2) XTG_GATE_HEADS(256, 4)
#undef XTG_GATE_HEADS
  HIP_CHECK(hipGetLastError());
  return strf("attn_gate_heads_kernel<%d, %d>", p.d, w);
}

std::string launch_attn_merge_heads(const AttnPlan& p, int n_q, int heads, const float* part, float* out,
                                    hipStream_t stream) {
  XTG_CHECK(p.blocks == 1 && n_q >= 1 && n_q <= p.rpb, "attention merge by heads: %d rows in %d blocks", n_q,
            p.blocks);
  XTG_CHECK(p.d == 64 || p.d == 128 || p.d == 256, "attention merge by heads: head_dim %d", p.d);
  XTG_CHECK(reinterpret_cast<uintptr_t>(out) % 16 == 0, "attention merge by heads: 16-byte aligned out");
  const MergeArgs a = merge_args(p, heads, part);
  const int w = merge_heads_waves(p, a.splits1);
  const dim3 grid{unsigned(heads), unsigned(n_q)}, block{unsigned(64 * w)};
#define XTG_MERGE_HEADS(D, W)                                                                                 \
  if (p.d == D && w == W)                                                                                     \
    hipLaunchKernelGGL((attn_merge_heads_kernel<D, W>), grid, block, 0, stream, a, out);
  XTG_MERGE_HEADS(64, 1) XTG_MERGE_HEADS(64, 2) XTG_MERGE_HEADS(64, 4)
  XTG_MERGE_HEADS(128, 1) XTG_MERGE_HEADS(128, 2) XTG_MERGE_HEADS(128, 4)
  XTG_MERGE_HEADS(256, 1) XTG_MERGE_HEADS(256, 2) XTG_MERGE_HEADS(256, 4)
#undef XTG_MERGE_HEADS
  HIP_CHECK(hipGetLastError());
  return strf("attn_merge_heads_kernel<%d, %d>", p.d, w);
}

}  // namespace xtg::hip
