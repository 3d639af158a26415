// Decode attention over a device-resident KV cache, and the cache's store.
//
// Semantics (engine/src/kv.cpp:166-286, npu/xtg_npu.cpp:236-258): query row i of this call (position pos0 + i)
// attends, for each of its q heads, to the cached keys whose stored position q satisfies 0 <= q < pos0 and
// (window <= 0 or pos0 + i - q < window), and to this call's own keys j <= i (with i - j < window); FP32 softmax of
// scale * q.k; the cache is read only. For a linear cache the stored position of slot s is s; for a ring it is
// whatever position was last written there (the slot-position array), so the mask is rebuilt from slot
// positions on every call.
//
// Device cache layout (head-major, in matrix-core operand order, slots padded to a multiple of 32):
//   K: per head, per block of 16 slots, per 32-wide chunk c of head_dim: 64 lanes x 8 BF16, lane (g, i) holding
//      slot 16 b + i, dims 32 c + 8 g .. +8: the A operand of v_mfma_f32_16x16x32_bf16 (keys x dims).
//   V: per head, per tile of 32 slots, per 16-wide block dd of head_dim: 64 lanes x 8 BF16, lane (g, i) holding
//      dim 16 dd + i of slots {4 g .. 4 g + 3, 16 + 4 g .. 16 + 4 g + 3}: the A operand (dims x keys) of the P.V
//      product whose B operand (keys x queries) is exactly what each lane holds of the score tile's accumulator.
//   slot_pos: int32 per slot, -1 = never written.
// Scores: S^T = K Q^T with the q vectors (times scale) split into three BF16 terms (about 24 significant bits, so
// sharp softmaxes keep FP32-level scores); K is BF16 and exact. P.V with P split into two BF16 terms. The q heads
// sharing a KV head and the query rows are stacked as MFMA columns (q-col = row * group + head), so every K and V
// byte is read once per KV head. This call's own keys (FP32, not yet stored) are added in FP32 on the vector ALUs.
// Flash decoding: a work-group of 4 waves per (KV head, split of the key tiles); the waves' online-softmax states
// are merged in LDS into one partial (max, sum, accumulator) per q-col, and attn_merge_kernel combines the splits.
#include <algorithm>
#include <cfloat>
#include <cmath>

#include "attention.hpp"
#include "common.hpp"

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

size_t kv_k_index(int h, int slot, int dim, int slots_pad, int d) { return k_index(h, slot, dim, slots_pad, d); }
size_t kv_v_index(int h, int slot, int dim, int slots_pad, int d) { return v_index(h, slot, dim, slots_pad, d); }

__device__ inline uint16_t f32_to_bf16_bits(float f) {
  // round to nearest even; a NaN stays a quiet NaN (engine/include/xtg/fp.h:18-24)
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return uint16_t((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

__device__ inline float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

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

void launch_kv_store(const DevKv& c, long long pos, int n, const float* k, const float* v, hipStream_t stream) {
  int first = 0;
  if (c.ring && n > c.slots) first = int(n - c.slots);
  const long long total = (long long)(n - first) * c.kv_heads * c.head_dim;
  if (total <= 0) return;
  const unsigned blocks = unsigned((total + 255) / 256);
  hipLaunchKernelGGL(kv_store_kernel, dim3(blocks), dim3(256), 0, stream, k, v, c.k, c.v, c.slot_pos, pos, first, n,
                     c.kv_heads, c.head_dim, (long long)c.slots, c.ring ? 1 : 0, c.slots_pad);
  HIP_CHECK(hipGetLastError());
}

// -------------------------------------------------------------------------------------------------- attention

struct AttnKernelArgs {
  const float* q;         // [n_rows][heads][d]: rows row0 .. row0 + n_rows - 1 of the call
  const float* k;         // [n_own][kv_heads][d] all of this call's keys (positions pos0 .. pos0 + n_own - 1)
  const float* v;
  const uint4* ck;        // cache, operand layout
  const uint4* cv;
  const int* slot_pos;
  float* part;            // [kv_heads][splits][qcols][2 + d]
  int n_rows, row0, n_own, heads, kv_heads, group, window, splits, slots_pad;
  int tile_lo, tiles;     // the key tiles to scan: tile_lo .. tile_lo + tiles - 1
  long long pos0;
  float scale;
};

__device__ inline bf16x8 bf16x8_of(const float v[8]) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = __builtin_bit_cast(__bf16, f32_to_bf16_bits(v[e]));
  return r;
}

// x = t0 + t1 + t2 + O(2^-24 |x|), each term the BF16 rounding of what is left.
__device__ inline void split3(const float x[8], bf16x8& t0, bf16x8& t1, bf16x8& t2) {
  float a[8], b[8], c[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = bf16_bits_to_f32(f32_to_bf16_bits(x[e]));
    const float r = x[e] - a[e];
    b[e] = bf16_bits_to_f32(f32_to_bf16_bits(r));
    c[e] = r - b[e];
  }
  t0 = bf16x8_of(a);
  t1 = bf16x8_of(b);
  t2 = bf16x8_of(c);
}

template <int D, int QB>
__global__ void __launch_bounds__(kWaves * 64) attn_decode_kernel(const AttnKernelArgs a) {
  constexpr int NC = D / 32;   // 32-dim chunks (QK^T contraction)
  constexpr int ND = D / 16;   // 16-dim blocks (P.V rows)
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int kvh = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
  const int qcols = a.n_rows * a.group;

  // q operands: column j of q-block qb is q-col qb * 16 + j = (row, head in the group); times scale, three terms
  bf16x8 qop[QB][NC][3];
  int qrow[QB];
  bool qlive[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qc = qb * 16 + j;
    qlive[qb] = qc < qcols;
    qrow[qb] = qlive[qb] ? qc / a.group : 0;
    const float* qp = a.q + (size_t(qrow[qb]) * size_t(a.heads) + size_t(kvh * a.group + (qlive[qb] ? qc % a.group : 0))) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float x[8];
      if (qlive[qb]) {
        const float4 u = *reinterpret_cast<const float4*>(qp + 32 * c + 8 * g);
        const float4 w = *reinterpret_cast<const float4*>(qp + 32 * c + 8 * g + 4);
        x[0] = u.x, x[1] = u.y, x[2] = u.z, x[3] = u.w, x[4] = w.x, x[5] = w.y, x[6] = w.z, x[7] = w.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= a.scale;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      }
      split3(x, qop[qb][c][0], qop[qb][c][1], qop[qb][c][2]);
    }
  }

  // online-softmax state of the lane's column in each q-block (the same in the 4 lanes of a column)
  float m[QB], l[QB];
  f32x4 acc[QB][ND];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
#pragma unroll
    for (int dd = 0; dd < ND; ++dd) acc[qb][dd] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // this split's tiles, dealt to the waves round-robin
  const int t_begin = a.tile_lo + int((long long)a.tiles * split / a.splits);
  const int t_end = a.tile_lo + int((long long)a.tiles * (split + 1) / a.splits);
  const size_t ktile = size_t(2 * NC) * 64, vtile = size_t(ND) * 64;   // uint4 per tile
  const uint4* kbase = a.ck + size_t(kvh) * size_t(a.slots_pad / kTile) * ktile;
  const uint4* vbase = a.cv + size_t(kvh) * size_t(a.slots_pad / kTile) * vtile;
  for (int t = t_begin + wave; t < t_end; t += kWaves) {
    uint4 kop[2][NC], vop[ND];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < NC; ++c) kop[b][c] = kbase[size_t(t) * ktile + size_t(b * NC + c) * 64 + size_t(lane)];
#pragma unroll
    for (int dd = 0; dd < ND; ++dd) vop[dd] = vbase[size_t(t) * vtile + size_t(dd) * 64 + size_t(lane)];
    const int4 p0 = *reinterpret_cast<const int4*>(a.slot_pos + t * kTile + 4 * g);
    const int4 p1 = *reinterpret_cast<const int4*>(a.slot_pos + t * kTile + 16 + 4 * g);
    const int kpos[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      f32x4 s[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        s[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8 A = __builtin_bit_cast(bf16x8, kop[b][c]);
#pragma unroll
          for (int term = 0; term < 3; ++term)
            s[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, qop[qb][c][term], s[b], 0, 0, 0);
        }
      }
      // mask, tile max over the lane's 8 keys and the column's 4 lanes
      const long long qpos = a.pos0 + a.row0 + qrow[qb];
      float sc[8];
      float mx = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kp = kpos[e];
        const bool see = qlive[qb] && kp >= 0 && kp < a.pos0 && (a.window <= 0 || qpos - kp < a.window);
        sc[e] = see ? s[e >> 2][e & 3] : -INFINITY;
        mx = fmaxf(mx, sc[e]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // No branch on visibility: every lane takes part in the shuffles and matrix ops below. A column with
      // nothing visible yet keeps max -inf, sum 0 and a zero accumulator (correction 1, probabilities 0).
      const float m_new = fmaxf(m[qb], mx);
      const float corr = m[qb] == -INFINITY ? (m_new == -INFINITY ? 1.f : 0.f) : expf(m[qb] - m_new);
      float p[8], ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = sc[e] == -INFINITY ? 0.f : expf(sc[e] - m_new);
        ps += p[e];
      }
      ps += __shfl_xor(ps, 16);
      ps += __shfl_xor(ps, 32);
      l[qb] = l[qb] * corr + ps;
      m[qb] = m_new;
      bf16x8 phi, plo;
      {
        float hi[8], lo[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hi[e] = bf16_bits_to_f32(f32_to_bf16_bits(p[e]));
          lo[e] = p[e] - hi[e];
        }
        phi = bf16x8_of(hi);
        plo = bf16x8_of(lo);
      }
#pragma unroll
      for (int dd = 0; dd < ND; ++dd) {
        acc[qb][dd] *= corr;
        const bf16x8 A = __builtin_bit_cast(bf16x8, vop[dd]);
        acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, phi, acc[qb][dd], 0, 0, 0);
        acc[qb][dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, plo, acc[qb][dd], 0, 0, 0);
      }
    }
  }

  // this call's own keys, in FP32: the last split's first wave
  if (split == a.splits - 1 && wave == 0) {
    for (int jj = 0; jj < a.n_own; ++jj) {
      const float* kr = a.k + (size_t(jj) * size_t(a.kv_heads) + size_t(kvh)) * D;
      const float* vr = a.v + (size_t(jj) * size_t(a.kv_heads) + size_t(kvh)) * D;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int qc = qb * 16 + j;
        const int hg = qlive[qb] ? qc % a.group : 0;
        const float* qp = a.q + (size_t(qrow[qb]) * size_t(a.heads) + size_t(kvh * a.group + hg)) * D;
        float dot = 0.f;
        for (int e = 0; e < D / 4; ++e) dot += qp[g * (D / 4) + e] * kr[g * (D / 4) + e];
        dot += __shfl_xor(dot, 16);
        dot += __shfl_xor(dot, 32);
        const int i = a.row0 + qrow[qb];   // the row's index in the call: it sees own keys jj <= i
        const bool see = qlive[qb] && jj <= i && (a.window <= 0 || i - jj < a.window);
        const float sc = see ? dot * a.scale : -INFINITY;
        const float m_new = fmaxf(m[qb], sc);
        const float corr = m[qb] == -INFINITY ? (m_new == -INFINITY ? 1.f : 0.f) : expf(m[qb] - m_new);
        const float pw = see ? expf(sc - m_new) : 0.f;
        l[qb] = l[qb] * corr + pw;
        m[qb] = m_new;
#pragma unroll
        for (int dd = 0; dd < ND; ++dd) {
          const float4 vv = *reinterpret_cast<const float4*>(vr + 16 * dd + 4 * g);
          acc[qb][dd][0] = acc[qb][dd][0] * corr + pw * vv.x;
          acc[qb][dd][1] = acc[qb][dd][1] * corr + pw * vv.y;
          acc[qb][dd][2] = acc[qb][dd][2] * corr + pw * vv.z;
          acc[qb][dd][3] = acc[qb][dd][3] * corr + pw * vv.w;
        }
      }
    }
  }

  // merge the 4 waves' states in LDS: [wave][qb][2 + D][16 cols] ... laid out as ml: [wave][qb][2][16], then
  // accumulators [wave][qb][dd][64 lanes][4]
  float* ml = lds;
  float* accs = lds + kWaves * QB * 2 * 16;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    if (g == 0) {
      ml[((wave * QB + qb) * 2 + 0) * 16 + j] = m[qb];
      ml[((wave * QB + qb) * 2 + 1) * 16 + j] = l[qb];
    }
#pragma unroll
    for (int dd = 0; dd < ND; ++dd)
      *reinterpret_cast<f32x4*>(accs + ((size_t(wave * QB + qb) * ND + dd) * 64 + lane) * 4) = acc[qb][dd];
  }
  __syncthreads();
  // wave w finishes q-block w (and w + 4, ...): partial (max, sum, accumulator[D]) of each live q-col
  for (int qb = wave; qb < QB; qb += kWaves) {
    const int qc = qb * 16 + j;
    float M = -INFINITY;
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ml[((w * QB + qb) * 2 + 0) * 16 + j]);
    float L = 0.f, f[kWaves];
    for (int w = 0; w < kWaves; ++w) {
      const float mw = ml[((w * QB + qb) * 2 + 0) * 16 + j];
      f[w] = mw == -INFINITY ? 0.f : expf(mw - M);
      L += f[w] * ml[((w * QB + qb) * 2 + 1) * 16 + j];
    }
    if (qc >= qcols) continue;
    float* out = a.part + ((size_t(kvh) * a.splits + split) * size_t(QB * 16) + size_t(qc)) * (2 + D);
    if (g == 0) {
      out[0] = M;
      out[1] = L;
    }
    for (int dd = 0; dd < ND; ++dd) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < kWaves; ++w)
        s += f[w] * *reinterpret_cast<const f32x4*>(accs + ((size_t(w * QB + qb) * ND + dd) * 64 + lane) * 4);
      *reinterpret_cast<f32x4*>(out + 2 + 16 * dd + 4 * g) = s;
    }
  }
}

// One work-group (D threads) per (row, q head): the splits' partials into out[row][head][:]
// (engine/src/kv.cpp:262-285; a split with no visible key has max -inf and sum 0 and is skipped).
__global__ void attn_merge_kernel(const float* __restrict__ part, float* __restrict__ out, int heads, int group,
                                  int splits, int qcols_pad, int d) {
  const int row = blockIdx.x / heads, h = blockIdx.x % heads, t = threadIdx.x;
  const int kvh = h / group, qc = row * group + h % group;
  float M = -INFINITY;
  for (int s = 0; s < splits; ++s)
    M = fmaxf(M, part[((size_t(kvh) * splits + s) * size_t(qcols_pad) + size_t(qc)) * (2 + d)]);
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float* p = part + ((size_t(kvh) * splits + s) * size_t(qcols_pad) + size_t(qc)) * (2 + d);
    if (p[1] == 0.f || p[0] == -INFINITY) continue;
    const float w = expf(p[0] - M);
    L += w * p[1];
    acc += w * p[2 + t];
  }
  out[(size_t(row) * heads + h) * d + t] = L > 0.f ? acc / L : 0.f;
}

namespace {
using AttnFn = void (*)(const AttnKernelArgs);
AttnFn attn_fn(int d, int qb) {
#define XTG_CASE(D, Q) \
  if (d == D && qb == Q) return attn_decode_kernel<D, Q>;
  XTG_CASE(64, 1) XTG_CASE(64, 2) XTG_CASE(64, 3) XTG_CASE(64, 4)
  XTG_CASE(128, 1) XTG_CASE(128, 2) XTG_CASE(128, 3) XTG_CASE(128, 4)
#undef XTG_CASE
  return nullptr;
}
}  // namespace

size_t attn_part_floats(int kv_heads, int splits, int qcols_pad, int d) {
  return size_t(kv_heads) * size_t(splits) * size_t(qcols_pad) * size_t(2 + d);
}

AttnPlan attn_plan(const DevKv& c, int n_q, int heads, long long pos0, int window) {
  XTG_CHECK(c.head_dim == 64 || c.head_dim == 128, "attention: head_dim %d (64 or 128)", c.head_dim);
  XTG_CHECK(heads % c.kv_heads == 0, "attention: %d heads over %d KV heads", heads, c.kv_heads);
  const int group = heads / c.kv_heads;
  XTG_CHECK(group <= 8, "attention: %d query heads per KV head (at most 8)", group);
  XTG_CHECK(n_q >= 1 && n_q * group <= 64, "attention: %d rows x %d heads per KV head (at most 64 columns)", n_q, group);
  AttnPlan p;
  p.group = group;
  p.qb = (n_q * group + 15) / 16;
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
  // about 512 work-groups over the KV heads, at least one tile per wave where there is work
  const int want = std::max(1, 512 / c.kv_heads);
  p.splits = std::max(1, std::min(want, (p.tiles + kWaves - 1) / kWaves));
  p.splits = std::min(p.splits, 128);
  return p;
}

int attn_rows_per_block(int group) { return std::max(1, 32 / group); }

size_t attn_part_floats_max(const DevKv& c, int n_q, int heads, long long pos0, int window) {
  const int rows = std::min(n_q, attn_rows_per_block(heads / c.kv_heads));
  const AttnPlan p = attn_plan(c, rows, heads, pos0, window);
  return attn_part_floats(c.kv_heads, p.splits, p.qb * 16, c.head_dim);
}

std::string launch_attn_decode(const DevKv& c, const AttnPlan& p, const float* q, const float* k, const float* v,
                               int n_rows, int row0, int n_own, int heads, long long pos0, int window, float scale,
                               float* part, hipStream_t stream) {
  AttnKernelArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.ck = reinterpret_cast<const uint4*>(c.k);
  a.cv = reinterpret_cast<const uint4*>(c.v);
  a.slot_pos = c.slot_pos;
  a.part = part;
  a.n_rows = n_rows;
  a.row0 = row0;
  a.n_own = n_own;
  a.heads = heads;
  a.kv_heads = c.kv_heads;
  a.group = p.group;
  a.window = window;
  a.splits = p.splits;
  a.slots_pad = c.slots_pad;
  a.tile_lo = p.tile_lo;
  a.tiles = p.tiles;
  a.pos0 = pos0;
  a.scale = scale;
  AttnFn fn = attn_fn(c.head_dim, p.qb);
  XTG_CHECK(fn != nullptr, "attention: no kernel for head_dim %d and %d column blocks", c.head_dim, p.qb);
  const int nd = c.head_dim / 16;
  const size_t lds = (size_t(kWaves) * p.qb * 2 * 16 + size_t(kWaves) * p.qb * nd * 64 * 4) * sizeof(float);
  if (lds > 65536) {   // the wave merge needs more than the default 64 KiB of LDS (gfx950 has 160 KiB)
    static thread_local AttnFn raised[8] = {};
    bool done = false;
    for (AttnFn f : raised) done |= f == fn;
    if (!done) {
      HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    int(lds)));
      for (AttnFn& f : raised)
        if (!f) {
          f = fn;
          break;
        }
    }
  }
  hipLaunchKernelGGL(fn, dim3(unsigned(c.kv_heads * p.splits)), dim3(kWaves * 64), lds, stream, a);
  HIP_CHECK(hipGetLastError());
  return strf("attn_decode_kernel<%d, %d>", c.head_dim, p.qb);
}

std::string launch_attn_merge(const DevKv& c, const AttnPlan& p, int n_rows, int heads, const float* part, float* out,
                              hipStream_t stream) {
  hipLaunchKernelGGL(attn_merge_kernel, dim3(unsigned(n_rows * heads)), dim3(unsigned(c.head_dim)), 0, stream, part,
                     out, heads, p.group, p.splits, p.qb * 16, c.head_dim);
  HIP_CHECK(hipGetLastError());
  return "attn_merge_kernel";
}

}  // namespace xtg::hip
