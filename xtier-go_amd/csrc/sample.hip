// Sampling on the device: xtg::Sampler::sample (engine/src/sampler.cpp:40-94) for rows of logits, with the
// uniform draw made by the caller.
//
// Semantics, per row of n logits (temperature > 0; temperature <= 0 is argmax, argmax_kernel):
//   w_i = exp((l_i - max) / T) in FP32 (the reference's expression: (l_i - max) * (1 / T)), total = sum w (double);
//   candidates in the order "larger weight first, then smaller index" (more_likely, sampler.cpp:26-28);
//   top_k in (0, n): keep the first top_k, total = their sum;
//   else min_p > 0 or top_p < 1: the candidates are sorted (the reference sorts a head of 1024 and, when top_p
//     needs it, everything; the kept prefix is the same once it lies in the sorted part);
//   min_p > 0: keep the leading candidates with w >= min_p * w_first (at least one), total = their sum;
//   top_p < 1: keep the shortest prefix whose running sum reaches total * top_p (at least one), total = that sum;
//   r = u * total with u in [0, 1) drawn by the caller (std::uniform_real_distribution<double>(0, total) is
//     total * generate_canonical<double, 53>); the token is the first kept candidate whose running sum exceeds r
//     (index order when no filter applies), else the last kept.
// Double sums run over contiguous chunks per thread in order, and the chunk sums combine by a wave scan: equal to
// the reference's left-to-right sums up to double rounding (a token can differ only when r lies within ~1e-15 of
// a running-sum boundary).
//
// Design: one work-group of 1024 threads per row, everything in one launch, every pass over the row coalesced
// (element i to thread i mod 1024). Running sums in a fixed order -- index order, or the sorted order -- go by
// segments: each wave sums a contiguous segment, the segment sums run in order, and the wave whose segment holds
// the crossing walks it in tiles of 64 with a wave scan.
// With a filter, the candidates are the weights at or above a threshold tau that the kept prefix cannot go below:
// every thread keeps its 4 most likely (weight, index) pairs during the weight pass; their union (4096 pairs,
// sorted in LDS) gives tau -- its top_k-th value for top_k, the value where its running mass first reaches
// total * top_p * (1 + 1e-6) for top_p, the floor for min_p (max(floor, that) with both) -- since the union is a
// subset of the row, the row holds at least as much above tau. The candidates (at most kCand) are gathered, sorted
// in LDS and filtered. When more than kCand weights lie at or above tau (a broad distribution under top_p or
// min_p), the whole row is sorted instead by a stable LSD radix sort in scratch memory (8 passes of 4 bits,
// contiguous chunks per thread): slower, the same result.
#include <cfloat>
#include <climits>
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "rowops.hpp"

namespace xtg::hip {

namespace {
constexpr int kSampleThreads = 1024;

// Exclusive prefix of v over the work-group in thread order; every thread gets its own prefix and *all the total.
// A wave scan by shuffles, then the 16 wave totals in order. red: at least kSampleThreads / 64 + 1 entries.
template <typename T>
__device__ inline T block_exclusive(T v, T* red, T* all) {
  const int t = int(threadIdx.x), lane = t & 63, wave = t >> 6;
  T x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  __syncthreads();   // red may still be read by a previous call
  if (lane == 63) red[wave] = x;
  __syncthreads();
  if (t == 0) {
    T s = T(0);
    for (int i = 0; i < kSampleThreads / 64; ++i) {
      const T c = red[i];
      red[i] = s;
      s += c;
    }
    red[kSampleThreads / 64] = s;
  }
  __syncthreads();
  *all = red[kSampleThreads / 64];
  return red[wave] + x - v;
}

// Double sums across a wave on the vector ALUs: DPP within rows of 16 on the two 32-bit halves, then the gfx950
// permlane swaps; every lane ends with the same value.
template <int CTRL>
__device__ inline double dpp_d(double v) {
  const uint64_t b = __double_as_longlong(v);
  const uint32_t lo = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b)), CTRL, 0xF, 0xF, false));
  const uint32_t hi = uint32_t(__builtin_amdgcn_update_dpp(0, int(uint32_t(b >> 32)), CTRL, 0xF, 0xF, false));
  return __longlong_as_double(int64_t((uint64_t(hi) << 32) | lo));
}
__device__ inline double swap16_sum_d(double v) {
  const uint64_t b = __double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane16_swap(uint32_t(b), uint32_t(b), false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap(uint32_t(b >> 32), uint32_t(b >> 32), false, false);
  return __longlong_as_double(int64_t((uint64_t(hi[0]) << 32) | lo[0])) +
         __longlong_as_double(int64_t((uint64_t(hi[1]) << 32) | lo[1]));
}
__device__ inline double swap32_sum_d(double v) {
  const uint64_t b = __double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane32_swap(uint32_t(b), uint32_t(b), false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap(uint32_t(b >> 32), uint32_t(b >> 32), false, false);
  return __longlong_as_double(int64_t((uint64_t(hi[0]) << 32) | lo[0])) +
         __longlong_as_double(int64_t((uint64_t(hi[1]) << 32) | lo[1]));
}
__device__ inline double wave_sum_d(double v) {
  v += dpp_d<kDppXor1>(v);
  v += dpp_d<kDppXor2>(v);
  v += dpp_d<kDppHalfMirror>(v);
  v += dpp_d<kDppMirror>(v);
  return swap32_sum_d(swap16_sum_d(v));
}

// Candidate order (sampler.cpp:26-28): a before b iff a's weight is larger, or equal at a smaller index.
__device__ inline bool more_likely(float wa, int ia, float wb, int ib) { return wa > wb || (wa == wb && ia < ib); }

// Sum of wf(i) over i = b + lane, b + lane + 64, .. < e for one wave: loads eight at a time, every wave-sum on DPP.
template <typename WF>
__device__ inline double wave_range_sum(WF wf, int b, int e) {
  const int lane = int(threadIdx.x) & 63;
  double s = 0.0;
  for (int i0 = b + lane; i0 < e; i0 += 8 * 64) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + 64 * u < e ? wf(i0 + 64 * u) : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) s += double(v[u]);
  }
  return wave_sum_d(s);
}

// The first position i in [0, len) at which the running sum of wf(0 .. i) satisfies strict ? sum > r : sum >= r,
// or len when none does; *at_sum: that running sum (the whole sum when none). Three levels: 16 segments (a wave
// each), the crossing segment's 16 parts (a wave each), then the crossing part's tiles of 64 by one wave, the
// crossing tile scanned. The sums of each level run in order. red: >= 20 doubles, sel: LDS int.
template <typename WF>
__device__ inline int first_crossing(WF wf, int len, double r, bool strict, double* red, int* sel, double* at_sum) {
  const int t = int(threadIdx.x), lane = t & 63, wave = t >> 6;
  constexpr int NW = kSampleThreads / 64;
  auto crosses = [&](double c) { return strict ? c > r : c >= r; };
  // level 1 and 2: [lo, hi) split into NW parts of `part` elements; the first part whose running sum crosses
  int lo = 0, hi = len;
  double base = 0.0;
  for (int level = 0; level < 2; ++level) {
    const int part = ((hi - lo + NW - 1) / NW + 63) / 64 * 64;
    const int b = min(hi, lo + wave * part), e = min(hi, b + part);
    const double s = wave_range_sum(wf, b, e);
    __syncthreads();   // red / sel may still be read by a previous step
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (t == 0) {
      double c = base, nb = 0.0;
      int found = -1;
      for (int w = 0; w < NW; ++w) {
        const double nc = c + red[w];
        if (found < 0 && crosses(nc)) {
          found = w;
          nb = c;
        }
        c = nc;
      }
      red[NW] = c;
      red[NW + 1] = nb;
      *sel = found;
    }
    __syncthreads();
    const int found = *sel;
    if (found < 0) {   // no crossing: the whole range's running sum (a part found by the level above, rounded
      *at_sum = red[NW];   // otherwise here, ends at its last element)
      __syncthreads();
      return level == 0 ? len : max(hi - 1, 0);
    }
    base = red[NW + 1];
    const int nlo = min(hi, lo + found * part);
    hi = min(hi, nlo + part);
    lo = nlo;
  }
  // level 3: one wave walks [lo, hi) (at most 8 tiles of 64 for rows up to 131072) in tiles, eight loaded at once
  if (wave == 0) {
    int hit = -1;
    double hs = base;
    float tv[8];
    for (int i0 = lo; i0 < hi && hit < 0; i0 += 64) {
      const int i = i0 + lane;
      const int u = ((i0 - lo) >> 6) & 7;
      if (u == 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) tv[q] = i + 64 * q < hi ? wf(i + 64 * q) : 0.f;
      }
      float xv = tv[0];
#pragma unroll
      for (int q = 1; q < 8; ++q) xv = u == q ? tv[q] : xv;
      const double x0 = double(xv);
      const double ts = wave_sum_d(x0);
      if (crosses(base + ts)) {   // the crossing tile: its running sums
        double x = x0;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const double y = __shfl_up(x, o);
          if (lane >= o) x += y;
        }
        const double cum = base + x;
        const unsigned long long m = __ballot(i < hi && crosses(cum));
        const int l = m ? __ffsll(m) - 1 : min(63, hi - 1 - i0);
        hit = i0 + l;
        hs = __shfl(cum, l);
      } else {
        base += ts;
        hs = base;
      }
    }
    if (hit < 0) hit = max(hi - 1, 0);   // the part's sum crossed, its walk (rounded otherwise) did not
    if (lane == 0) {
      *sel = hit;
      red[NW + 2] = hs;
    }
  }
  __syncthreads();
  const int first = *sel;
  *at_sum = red[NW + 2];
  __syncthreads();
  return first;
}

// Bitonic sort of n2 (a power of two, <= kCand) pairs in LDS into candidate order; every thread of the work-group.
__device__ inline void sort_pairs(float* cw, int* ci, int n2) {
  for (int k = 2; k <= n2; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      __syncthreads();
      for (int p = int(threadIdx.x); p < n2 / 2; p += kSampleThreads) {
        const int lo = 2 * p - (p & (j - 1)), hi = lo + j;   // lo has bit j clear
        const bool up = (lo & k) == 0;                        // this run ascends in candidate order
        const float wl = cw[lo], wh = cw[hi];
        const int il = ci[lo], ih = ci[hi];
        if (more_likely(wh, ih, wl, il) == up) {
          cw[lo] = wh;
          cw[hi] = wl;
          ci[lo] = ih;
          ci[hi] = il;
        }
      }
    }
  __syncthreads();
}
}  // namespace

struct SampleArgs {
  const float* logits;   // [rows][n]
  int n;
  float temperature, top_p, min_p;
  int top_k;
  double u[kMaxSampleRows];
  float* w;              // scratch [rows][n]
  uint32_t* keys;        // scratch [rows][2][n]
  int* idx;              // scratch [rows][2][n]
  int* out;              // [rows]
};

constexpr int kCand = 4096;   // candidates sorted in LDS (the union of the threads' top 4 has this many)
constexpr int kTop = kCand / kSampleThreads;

__global__ void __launch_bounds__(kSampleThreads) sample_kernel(const SampleArgs a) {
  __shared__ double red[kSampleThreads / 64 + 4];   // >= 20
  __shared__ uint32_t ured[kSampleThreads / 64 + 1];
  __shared__ uint32_t hist[16 * kSampleThreads];   // the fallback sort's digit counts
  __shared__ float cw[kCand];
  __shared__ int ci[kCand];
  __shared__ float fmx[kSampleThreads / 64];
  __shared__ int sel, ccount;
  __shared__ float tau_s;
  const int row = int(blockIdx.x), t = int(threadIdx.x), n = a.n;
  const float* l = a.logits + size_t(row) * size_t(n);
  float* w = a.w + size_t(row) * size_t(n);

  // the largest logit (std::max order is immaterial for finite rows), the weights, their total, each thread's
  // 4 most likely, and (min_p) the count and mass at or above the floor min_p * w_max = min_p (w_max = exp(0))
  float mx = -INFINITY;
  for (int i0 = t; i0 < n; i0 += 8 * kSampleThreads) {   // eight loads in flight per thread
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + u * kSampleThreads < n ? l[i0 + u * kSampleThreads] : -INFINITY;
#pragma unroll
    for (int u = 0; u < 8; ++u) mx = fmaxf(mx, v[u]);
  }
  mx = wave_max(mx);
  if ((t & 63) == 0) fmx[t >> 6] = mx;
  __syncthreads();
  mx = fmx[0];
  for (int i = 1; i < kSampleThreads / 64; ++i) mx = fmaxf(mx, fmx[i]);
  const float inv_t = 1.f / a.temperature;
  const float floor_w = a.min_p * 1.0f;
  float tw[kTop];
  int ti[kTop];
#pragma unroll
  for (int q = 0; q < kTop; ++q) tw[q] = -1.f, ti[q] = INT_MAX;
  double s = 0.0, sfl = 0.0;
  int nfl = 0;
  for (int i0 = t; i0 < n; i0 += 8 * kSampleThreads) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = i0 + u * kSampleThreads < n ? l[i0 + u * kSampleThreads] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
    const int i = i0 + u * kSampleThreads;
    if (i >= n) break;
    const float x = expf((v[u] - mx) * inv_t);
    w[i] = x;
    s += double(x);
    if (x >= floor_w) {
      sfl += double(x);
      ++nfl;
    }
    if (more_likely(x, i, tw[kTop - 1], ti[kTop - 1])) {   // insert, keeping the list in candidate order
      float cwv = x;
      int civ = i;
#pragma unroll
      for (int q = 0; q < kTop; ++q)
        if (more_likely(cwv, civ, tw[q], ti[q])) {
          const float tv = tw[q];
          const int tiv = ti[q];
          tw[q] = cwv;
          ti[q] = civ;
          cwv = tv;
          civ = tiv;
        }
    }
    }
  }
  double total, t_floor;
  block_exclusive(s, red, &total);
  block_exclusive(sfl, red, &t_floor);
  uint32_t n_floor;
  block_exclusive<uint32_t>(uint32_t(nfl), ured, &n_floor);
  __syncthreads();   // w complete

  const bool topk = a.top_k > 0 && a.top_k < n;
  if (!topk && a.top_p >= 1.f && a.min_p <= 0.f) {   // no filter: the candidates in index order
    double at;
    const int i = first_crossing([&](int j) { return w[j]; }, n, a.u[row] * total, true, red, &sel, &at);
    if (t == 0) a.out[row] = i < n ? i : n - 1;
    return;
  }

  // tau from the union of the threads' top 4 (sorted): the kept prefix lies at or above it
#pragma unroll
  for (int q = 0; q < kTop; ++q) {
    cw[t * kTop + q] = tw[q];
    ci[t * kTop + q] = ti[q];
  }
  sort_pairs(cw, ci, kCand);
  if (t == 0) {
    float tau = 0.f;
    bool ok = true;
    if (topk) {
      ok = a.top_k <= kCand && cw[a.top_k - 1] >= 0.f;
      tau = ok ? cw[a.top_k - 1] : 0.f;
    } else {
      if (a.top_p < 1.f) {
        const double target = total * double(a.top_p) * (1.0 + 1e-6);
        double c = 0.0;
        int q = 0;
        while (q < kCand && cw[q] >= 0.f && c < target) c += double(cw[q++]);
        ok = c >= target;
        tau = ok ? cw[q - 1] : 0.f;
      }
      if (a.min_p > 0.f) tau = fmaxf(tau, floor_w);
    }
    tau_s = ok ? tau : -1.f;   // -1: no bound from the union
    ccount = 0;
  }
  __syncthreads();
  const float tau = tau_s;
  // gather the candidates w >= tau (order-free: they are sorted next)
  if (tau >= 0.f) {
    for (int i0 = t; i0 < n; i0 += 8 * kSampleThreads) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = i0 + u * kSampleThreads < n ? w[i0 + u * kSampleThreads] : -1.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (v[u] >= tau) {
          const int pos = atomicAdd(&ccount, 1);
          if (pos < kCand) {
            cw[pos] = v[u];
            ci[pos] = i0 + u * kSampleThreads;
          }
        }
    }
  }
  __syncthreads();
  const int nc = tau >= 0.f ? ccount : INT_MAX;
  __syncthreads();

  const float* sw_l = cw;
  const int* si_l = ci;
  const uint32_t* ksrc = nullptr;
  const int* isrc = nullptr;
  int L;   // candidates available in order
  if (nc <= kCand) {
    int n2 = 1;
    while (n2 < nc) n2 <<= 1;
    for (int q = nc + t; q < n2; q += kSampleThreads) {
      cw[q] = -1.f;
      ci[q] = INT_MAX;
    }
    sort_pairs(cw, ci, n2);
    L = nc;
  } else {
    // the whole row, stably sorted by (~bits(w), index), 4 bits a pass, contiguous chunks per thread
    uint32_t* k0 = a.keys + size_t(row) * 2 * size_t(n);
    uint32_t* k1 = k0 + n;
    int* i0 = a.idx + size_t(row) * 2 * size_t(n);
    int* i1 = i0 + n;
    const int chunk = (n + kSampleThreads - 1) / kSampleThreads;
    const int b = min(n, t * chunk), e = min(n, b + chunk);
    uint32_t* kr = k0;
    int* ir = i0;
    uint32_t* kw = k1;
    int* iw = i1;
    for (int pass = 0; pass < 8; ++pass) {
      const int sh = 4 * pass;
      uint32_t cnt[16];
#pragma unroll
      for (int d = 0; d < 16; ++d) cnt[d] = 0;
      for (int i = b; i < e; ++i) {
        const uint32_t key = pass == 0 ? ~__float_as_uint(w[i]) : kr[i];
        const uint32_t dg = (key >> sh) & 15u;
#pragma unroll
        for (int d = 0; d < 16; ++d) cnt[d] += dg == uint32_t(d) ? 1u : 0u;
      }
      __syncthreads();   // hist free (the previous pass's scatter is done reading it)
#pragma unroll
      for (int d = 0; d < 16; ++d) hist[d * kSampleThreads + t] = cnt[d];
      __syncthreads();
      // exclusive scan of hist in (digit, thread) order: thread t owns entries 16 t .. 16 t + 15
      uint32_t part = 0;
#pragma unroll
      for (int q = 0; q < 16; ++q) part += hist[16 * t + q];
      uint32_t tot_unused;
      uint32_t run = block_exclusive<uint32_t>(part, ured, &tot_unused);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const uint32_t c = hist[16 * t + q];
        hist[16 * t + q] = run;
        run += c;
      }
      __syncthreads();
      uint32_t off[16];
#pragma unroll
      for (int d = 0; d < 16; ++d) off[d] = hist[d * kSampleThreads + t];
      for (int i = b; i < e; ++i) {
        const uint32_t key = pass == 0 ? ~__float_as_uint(w[i]) : kr[i];
        const int id = pass == 0 ? i : ir[i];
        const uint32_t dg = (key >> sh) & 15u;
        uint32_t dst = 0;
#pragma unroll
        for (int d = 0; d < 16; ++d)
          if (dg == uint32_t(d)) dst = off[d]++;
        kw[dst] = key;
        iw[dst] = id;
      }
      __syncthreads();   // the pass's output is complete before the next reads it
      uint32_t* kt = kr;
      kr = kw;
      kw = pass == 0 ? k0 : kt;
      int* it = ir;
      ir = iw;
      iw = pass == 0 ? i0 : it;
    }
    ksrc = kr;
    isrc = ir;
    L = n;
  }
  auto sw = [&](int j) { return ksrc ? __uint_as_float(~ksrc[j]) : sw_l[j]; };
  auto sidx = [&](int j) { return ksrc ? isrc[j] : si_l[j]; };

  // the reference's filters over the candidates in order (sampler.cpp:63-91)
  int keep = n;
  double at;
  if (topk) {
    keep = a.top_k;
    first_crossing(sw, keep, INFINITY, true, red, &sel, &at);
    total = at;   // the sum of the first top_k
  }
  if (a.min_p > 0.f) {
    int k;
    double tk;
    if (topk || ksrc) {   // the leading candidates >= floor, a prefix of the order
      if (t == 0) sel = INT_MAX;
      __syncthreads();
      const int lim = min(keep, L);
      for (int i = t; i < lim; i += kSampleThreads)
        if (!(sw(i) >= floor_w)) atomicMin(&sel, i);
      __syncthreads();
      k = sel == INT_MAX ? lim : sel;
      __syncthreads();
      first_crossing(sw, k, INFINITY, true, red, &sel, &tk);
    } else {   // every weight >= floor: counted over the row in the weight pass
      k = int(n_floor);
      tk = t_floor;
    }
    keep = max(1, k);
    total = k ? tk : double(sw(0));
  }
  if (a.top_p < 1.f) {
    const double target = total * double(a.top_p);
    const int lim = min(keep, L);
    const int i = first_crossing(sw, lim, target, false, red, &sel, &at);
    keep = max(1, i < lim ? i + 1 : lim);
    total = at;
  }
  const int lim = min(keep, L);
  const int i = first_crossing(sw, lim, a.u[row] * total, true, red, &sel, &at);
  if (t == 0) a.out[row] = sidx(i < lim ? i : lim - 1);
}

size_t sample_scratch_bytes(int rows, int n) { return size_t(rows) * size_t(n) * (sizeof(float) + 4 * sizeof(uint32_t)); }

std::string launch_sample(const float* logits, int rows, int n, float temperature, float top_p, int top_k,
                          float min_p, const double* u, int* out, void* scratch, hipStream_t stream) {
  XTG_CHECK(rows >= 1 && rows <= kMaxSampleRows, "sample: %d rows (1..%d)", rows, kMaxSampleRows);
  XTG_CHECK(n >= 1, "sample: %d logits", n);
  XTG_CHECK(temperature > 0.f, "sample: temperature %g (greedy decoding is argmax)", double(temperature));
  SampleArgs a{};
  a.logits = logits;
  a.n = n;
  a.temperature = temperature;
  a.top_p = top_p;
  a.min_p = min_p;
  a.top_k = top_k;
  for (int r = 0; r < rows; ++r) {
    XTG_CHECK(u[r] >= 0.0 && u[r] < 1.0, "sample: draw %g outside [0, 1)", u[r]);
    a.u[r] = u[r];
  }
  a.w = static_cast<float*>(scratch);
  a.keys = reinterpret_cast<uint32_t*>(a.w + size_t(rows) * size_t(n));
  a.idx = reinterpret_cast<int*>(a.keys + size_t(rows) * 2 * size_t(n));
  a.out = out;
  hipLaunchKernelGGL(sample_kernel, dim3(unsigned(rows)), dim3(kSampleThreads), 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return "sample_kernel";
}

}  // namespace xtg::hip
