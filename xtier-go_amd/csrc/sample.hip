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
// Design: three launches. Slices of 2048 logits (a work-group of 256 each): their maxima; then, with the row's max,
// their weights, sums (fixed order), min_p counts and, with a filter, every thread's two most likely pairs (the
// slice's 64 largest thread maxima in candidate order, and the largest second). Then
// one work-group of 1024 threads per row: the slice sums in order give the total and, without a filter, the slice
// where the running sum passes r, walked by hierarchical running sums (16 wave segments, 16 parts, tiles of 64).
// With a filter, a threshold tau that the kept prefix cannot go below comes from the union of the slices' lists --
// for top_k up to 64 its top_k-th pair (merges that keep the first 64); for a larger top_k, and for top_p, the lower
// edge of the 24-bit bucket of weight bits where the union's running count reaches top_k, or its mass total * top_p
// * (1 + 1e-6) (a radix select, three passes of 256 counters; masses in fixed point, so exact and order-free); the
// floor for min_p (max(floor, that) with both): the union is a subset of the row, so the row holds at least as much
// at or above tau. When in every slice the 64th listed maximum and every thread's second lie below tau, the union
// holds every weight >= tau, and the candidates are its pairs at or above tau; otherwise they are gathered from
// the row (at most 4096, sorted in LDS), or, past that, the whole row is sorted by a stable LSD radix sort in scratch
// memory (8 passes of 4 bits): slower, the same result. Sorts in LDS are merges of sorted runs of 64 (the slices'
// lists as they come; gathered pairs sorted by the waves in registers first), one barrier per doubling of the run
// instead of one per stage of a bitonic network over the whole set (78 for 4096 pairs). Greedy rows take the
// slices' first maxima (argmax_pick_kernel).
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
// A wave scan by shuffles, then every thread adds the 16 wave totals before its wave (in order) itself. red: at
// least kSampleThreads / 64 entries.
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
  T before = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < kSampleThreads / 64; ++i) {
    const T c = red[i];
    before += i < wave ? c : T(0);
    tot += c;
  }
  *all = tot;
  return before + x - v;
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
// or len when none does; *at_sum: that running sum (the whole sum when none), both counted from base0. Up to three
// levels: 16 segments (a wave each), the crossing segment's 16 parts (a wave each) unless the segment holds at most
// 512, then the crossing range's tiles of 64 by one wave, the crossing tile scanned. The sums of each level run in
// order. red: >= 20 doubles, sel: LDS int.
template <typename WF>
__device__ inline int first_crossing(WF wf, int len, double r, bool strict, double* red, int* sel, double* at_sum,
                                     double base0 = 0.0) {
  const int t = int(threadIdx.x), lane = t & 63, wave = t >> 6;
  constexpr int NW = kSampleThreads / 64;
  auto crosses = [&](double c) { return strict ? c > r : c >= r; };
  // level 1 and 2: [lo, hi) split into NW parts of `part` elements; the first part whose running sum (from base0)
  // crosses
  int lo = 0, hi = len;
  double base = base0;
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
    if (hi - lo <= 512) break;   // few enough for the walk below (8 tiles of 64 loaded at once)
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

// Candidate order over (weight, index) pairs is total for distinct indices (the padding pairs (-1, INT_MAX) are
// equal to each other), so every sort below gives the one order a sort of the reference's comparator gives. In LDS
// a pair is one 64-bit key whose ascending order is candidate order: above, the weight's bits mapped so that larger
// weights give smaller values (desc_key); below, the index. Weights >= 0 sort before the padding's -1.
__device__ inline uint32_t desc_key(float w) {
  const uint32_t u = __float_as_uint(w);
  return ~(u ^ ((u >> 31) ? 0xffffffffu : 0x80000000u));
}
__device__ inline unsigned long long pair_key(float w, int id) {
  return (static_cast<unsigned long long>(desc_key(w)) << 32) | uint32_t(id);
}
constexpr unsigned long long kPadKey = 0xbf8000007fffffffull;   // pair_key(-1, INT_MAX)
__device__ inline float key_w(unsigned long long k) {
  const uint32_t y = ~uint32_t(k >> 32);
  return __uint_as_float((y & 0x80000000u) ? (y ^ 0x80000000u) : ~y);
}
__device__ inline int key_id(unsigned long long k) { return int(uint32_t(k)); }

// One wave's key in lane l of a run of 64 sorted in registers into ascending order (lane 0 most likely): a bitonic
// network over the lanes (partner l ^ j by shuffle), every run of 2k ascending where l & k is clear, the last level
// all ascending. Equal keys stay where they are.
__device__ inline void wave_sort64(unsigned long long& k) {
  const int l = int(threadIdx.x) & 63;
#pragma unroll
  for (int r = 2; r <= 64; r <<= 1)
#pragma unroll
    for (int j = r >> 1; j > 0; j >>= 1) {
      const unsigned long long kp = __shfl_xor(k, j);
      const bool up = r == 64 || (l & r) == 0;   // this run ascends
      const bool first = (l & j) == 0;            // the lower place of the pair
      // the lower place of an ascending run (the upper of a descending one) takes the smaller key
      const bool take = up == first ? kp < k : k < kp;
      if (take) k = kp;
    }
}

// n2 (a power of two) keys in LDS whose runs of `run` keys (a power of two) are each ascending, merged into ascending
// order by pairwise merges of the runs, one level per doubling. Each thread makes E = n2 / NT consecutive outputs
// of its pair of runs (A, B), at least one: it finds by binary search on its diagonal how many of A's keys come
// before its first output (merge path), then merges E keys in order; of two equal keys A's goes first. tk: scratch
// for n2 keys. The result is in ck; every thread of the work-group (NT) takes part.
template <int NT>
__device__ inline void merge_runs(unsigned long long* ck, unsigned long long* tk, int n2, int run) {
  const int E = n2 > NT ? n2 / NT : 1;
  unsigned long long* src = ck;
  unsigned long long* dst = tk;
  for (int L = run; L < n2; L <<= 1) {
    __syncthreads();
    const int o0 = int(threadIdx.x) * E;
    if (o0 < n2) {
      const int base = o0 & ~(2 * L - 1), d = o0 - base;
      const unsigned long long* A = src + base;
      const unsigned long long* B = A + L;
      int lo = d > L ? d - L : 0, hi = d < L ? d : L;
      while (lo < hi) {   // A's keys among the first d outputs: A[mid] goes first unless B[d - 1 - mid] is smaller
        const int mid = (lo + hi) >> 1;
        if (B[d - 1 - mid] < A[mid])
          hi = mid;
        else
          lo = mid + 1;
      }
      int x = lo, y = d - lo;
      unsigned long long ka = x < L ? A[x] : ~0ull, kb = y < L ? B[y] : ~0ull;
      for (int e = 0; e < E; ++e) {
        const bool take_a = ka <= kb;   // an exhausted run reads as the largest key
        dst[o0 + e] = take_a ? ka : kb;
        if (take_a)
          ka = ++x < L ? A[x] : ~0ull;
        else
          kb = ++y < L ? B[y] : ~0ull;
      }
    }
    unsigned long long* tmp = src;
    src = dst;
    dst = tmp;
  }
  __syncthreads();
  if (src != ck) {   // an odd number of levels: the result back into ck
    for (int q = int(threadIdx.x); q < n2; q += NT) ck[q] = src[q];
    __syncthreads();
  }
}

// The R smallest of nr ascending runs of R keys each (nr and R powers of two), in order, into ck[0, R): pairwise
// merges that keep each pair's first R, one level per halving of the runs (output d of a pair by merge path on
// diagonal d, A's key first of two equal ones). tk: scratch for nr R / 2 keys. Every thread of the work-group (NT).
template <int NT>
__device__ inline void merge_top(unsigned long long* ck, unsigned long long* tk, int nr, int R) {
  unsigned long long* src = ck;
  unsigned long long* dst = tk;
  for (int m = nr; m > 1; m >>= 1) {
    __syncthreads();
    for (int q = int(threadIdx.x); q < (m >> 1) * R; q += NT) {
      const int pr = q / R, d = q - pr * R;
      const unsigned long long* A = src + 2 * pr * R;
      const unsigned long long* B = A + R;
      int lo = 0, hi = d;   // d < R: both runs can supply all d
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (B[d - 1 - mid] < A[mid])
          hi = mid;
        else
          lo = mid + 1;
      }
      const unsigned long long ka = A[lo], kb = B[d - lo];   // lo, d - lo < R
      dst[q] = ka <= kb ? ka : kb;
    }
    unsigned long long* tmp = src;
    src = dst;
    dst = tmp;
  }
  __syncthreads();
  if (src != ck) {
    for (int q = int(threadIdx.x); q < R; q += NT) ck[q] = src[q];
    __syncthreads();
  }
}

// n2 (a power of two, <= kCand) keys in LDS in any order into ascending order: runs of 64 sorted by the waves in
// registers, then merged. tk: scratch for n2 keys. Every thread of the work-group (NT threads).
template <int NT>
__device__ inline void sort_pairs(unsigned long long* ck, unsigned long long* tk, int n2) {
  const int lane = int(threadIdx.x) & 63, wave = int(threadIdx.x) >> 6;
  __syncthreads();   // the keys are in
  for (int r = wave; r * 64 < n2; r += NT / 64) {
    const int q = r * 64 + lane;
    unsigned long long k = q < n2 ? ck[q] : kPadKey;   // a run shorter than 64 (n2 < 64): padding that sorts last
    wave_sort64(k);
    if (q < n2) ck[q] = k;
  }
  merge_runs<NT>(ck, tk, n2, n2 < 64 ? n2 : 64);
}

// A weight that the kept prefix cannot go below, from the U pairs of the slices' lists (weights in [0, 1]; below 0:
// padding): an MSD radix select over the weights' bits, 8 a pass for three passes, finds the bucket of 24 leading
// bits in which the running count (mass = false) or mass of the union from its most likely side first reaches
// `target` (<= U; a mass target < U), and returns the bucket's lower edge; -1 when the union never reaches it. Masses are fixed point
// at 2^-F with U <= 2^(62 - F): the sums are exact and order-free, each weight's share is rounded down and the
// target up. The row holds the union, so its own count or mass at or above that edge is at least as large. h: 256
// LDS counters; sel, above: LDS words. Every thread of the work-group.
__device__ inline float union_select(const float* __restrict__ uw, int U, bool mass, double target,
                                     unsigned long long* h, int* sel, unsigned long long* above_s) {
  const int t = int(threadIdx.x), lane = t & 63, wave = t >> 6;
  const double scale = ldexp(1.0, 62 - (32 - __clz(U)));
  const unsigned long long tgt = mass ? (unsigned long long)ceil(target * scale) : (unsigned long long)target;
  uint32_t prefix = 0u;
  unsigned long long above = 0ull;
  // the first 4 * kSampleThreads weights stay in registers over the passes (the lists were written on other XCDs:
  // each read waits on memory); any beyond are read again by each pass
  constexpr int KR = 4;
  float xr[KR];
#pragma unroll
  for (int r = 0; r < KR; ++r) {
    const int e = t + r * kSampleThreads;
    xr[r] = e < U ? uw[e] : -1.f;
  }
  for (int p = 0; p < 3; ++p) {
    const int sh = 24 - 8 * p;
    if (t < 256) h[t] = 0ull;
    __syncthreads();
    auto add = [&](float x) {
      const uint32_t b = __float_as_uint(x);
      if (x >= 0.f && (p == 0 || (b >> (sh + 8)) == prefix))
        atomicAdd(&h[(b >> sh) & 255u], mass ? (unsigned long long)(double(x) * scale) : 1ull);
    };
#pragma unroll
    for (int r = 0; r < KR; ++r) add(xr[r]);
    for (int e = t + KR * kSampleThreads; e < U; e += kSampleThreads) add(uw[e]);
    __syncthreads();
    if (wave == 0) {   // digits from the most likely: lane l holds 255 - 4 l .. 252 - 4 l
      unsigned long long c[4], s = 0ull;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = h[255 - 4 * lane - q];
        s += c[q];
      }
      unsigned long long x = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      const unsigned long long m = __ballot(above + x >= tgt);
      const int l = m ? __ffsll(m) - 1 : 0;
      if (lane == l) {
        int d = -1;
        unsigned long long run = above + x - s;
        if (m) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (d < 0) {
              if (run + c[q] >= tgt)
                d = 255 - 4 * lane - q;
              else
                run += c[q];
            }
          }
        }
        *sel = d;
        *above_s = run;
      }
    }
    __syncthreads();
    const int d = *sel;
    above = *above_s;
    __syncthreads();   // sel, above_s and h are written again by the next pass or the caller
    if (d < 0) return -1.f;
    prefix = (prefix << 8) | uint32_t(d);
  }
  return __uint_as_float(prefix << 8);
}
}  // namespace

// Per-row scratch (floats / ints / doubles laid out by SampleScratch): the weights, and per slice of kSlice logits
// its max, argmax, weight sum, count and mass at or above the min_p floor, its 64 largest thread maxima in
// candidate order (-1 weights past the slice's threads) and the largest second-most-likely weight of a thread.
constexpr int kSlice = 2048, kSliceThreads = 256, kSliceTop = 64;
constexpr int kCand = 4096;   // candidates sorted in LDS

struct SampleArgs {
  const float* logits;   // [rows][n]
  int n, slices;
  float temperature, top_p, min_p;
  int top_k;
  double u[kMaxSampleRows];
  float* w;              // [rows][n]
  float* smax;           // [rows][slices]
  float* sbest;          // [rows][slices] argmax value, index in sbi
  int* sbi;
  double* ssum;          // [rows][slices]
  double* sfl;           // [rows][slices] mass >= floor
  int* snfl;             // [rows][slices] count >= floor
  float* sw;             // [rows][slices][kSliceTop]: the slice's 64 largest thread maxima, in candidate order
  int* si;
  float* sm2;            // [rows][slices]: the largest second-most-likely weight of any thread of the slice
  float* tmax;           // [rows][slices][kSliceThreads]: each slice thread's most likely weight (-1: none)
  float* tsec;           // [rows][slices][kSliceThreads]: its second most likely (-1: none)
  uint8_t* tu;           // [rows][slices][kSliceThreads]: the most likely one's place u (index b + t + 256 u)
  int lists;             // a filter applies: make the lists
  uint32_t* keys;        // [rows][2][n] (the whole-row sort)
  int* idx;
  int* out;              // [rows]
};

// Slice maxima (the weights' reference point) and, for greedy decoding, each slice's first largest finite-or-inf
// value (NaNs never win: xtg::argmax, sampler.cpp:8-13).
__global__ void __launch_bounds__(kSliceThreads) slice_max_kernel(const SampleArgs a) {
  __shared__ float sv[kSliceThreads / 64];
  __shared__ int sx[kSliceThreads / 64];
  __shared__ float sm[kSliceThreads / 64];
  const int row = int(blockIdx.y), sl = int(blockIdx.x), t = int(threadIdx.x);
  const float* l = a.logits + size_t(row) * size_t(a.n);
  const int b = sl * kSlice, e = min(a.n, b + kSlice);
  float v[kSlice / kSliceThreads];
#pragma unroll
  for (int u = 0; u < kSlice / kSliceThreads; ++u) {
    const int i = b + t + u * kSliceThreads;
    v[u] = i < e ? l[i] : -INFINITY;
  }
  float mx = -INFINITY, bv = -INFINITY;
  int bi = INT_MAX;
#pragma unroll
  for (int u = 0; u < kSlice / kSliceThreads; ++u) {
    const int i = b + t + u * kSliceThreads;
    mx = fmaxf(mx, v[u]);
    if (i < e && (v[u] > bv || (v[u] == bv && i < bi))) bv = v[u], bi = i;
  }
  mx = wave_max(mx);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) bv = ov, bi = oi;
  }
  if ((t & 63) == 0) sv[t >> 6] = bv, sx[t >> 6] = bi, sm[t >> 6] = mx;
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kSliceThreads / 64; ++w) {
      if (sv[w] > bv || (sv[w] == bv && sx[w] < bi)) bv = sv[w], bi = sx[w];
      mx = fmaxf(mx, sm[w]);
    }
    a.smax[size_t(row) * a.slices + sl] = mx;
    a.sbest[size_t(row) * a.slices + sl] = bv;
    a.sbi[size_t(row) * a.slices + sl] = bi;
  }
}

// The first largest over the slices (a NaN in element 0, or no element above -inf that is not NaN, gives 0).
__global__ void __launch_bounds__(64) argmax_pick_kernel(const SampleArgs a) {
  const int row = int(blockIdx.x), t = int(threadIdx.x);
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int s = t; s < a.slices; s += 64) {
    const float v = a.sbest[size_t(row) * a.slices + s];
    const int i = a.sbi[size_t(row) * a.slices + s];
    if (i != INT_MAX && (v > bv || (v == bv && i < bi))) bv = v, bi = i;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (oi != INT_MAX && (ov > bv || (ov == bv && oi < bi) || bi == INT_MAX)) bv = ov, bi = oi;
  }
  if (t == 0) {
    const float x0 = a.logits[size_t(row) * size_t(a.n)];
    a.out[row] = (x0 != x0 || bi == INT_MAX) ? 0 : bi;
  }
}

// The slice's weights w = expf((l - max) * (1 / T)) (max over every slice), their sum in a fixed order, the count
// and mass at or above the min_p floor (min_p * w_max, w_max = exp(0) = 1), and (with a filter) every thread's two
// most likely pairs: the 64 largest of the threads' first ones in candidate order (256 sorted in LDS) and the
// largest of their second ones. Any weight of the slice at or above a threshold above both is one of those 64.
__global__ void __launch_bounds__(kSliceThreads) slice_weights_kernel(const SampleArgs a) {
  __shared__ unsigned long long ck[kSliceThreads], tk[kSliceThreads];
  __shared__ double dred[kSliceThreads / 64][2];
  __shared__ int ired[kSliceThreads / 64];
  __shared__ float m2red[kSliceThreads / 64];
  const int row = int(blockIdx.y), sl = int(blockIdx.x), t = int(threadIdx.x);
  const float* l = a.logits + size_t(row) * size_t(a.n);
  float* w = a.w + size_t(row) * size_t(a.n);
  const int b = sl * kSlice, e = min(a.n, b + kSlice);
  // the row's max over the slices' maxima: loaded in parallel (they were written on other XCDs), then reduced
  __shared__ float mred[kSliceThreads / 64];
  float mx = -INFINITY;
  for (int s = t; s < a.slices; s += kSliceThreads) mx = fmaxf(mx, a.smax[size_t(row) * a.slices + s]);
  mx = wave_max(mx);
  if ((t & 63) == 0) mred[t >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kSliceThreads / 64; ++q) mx = fmaxf(mx, mred[q]);
  const float inv_t = 1.f / a.temperature;
  const float floor_w = a.min_p * 1.0f;
  float v[kSlice / kSliceThreads];
#pragma unroll
  for (int u = 0; u < kSlice / kSliceThreads; ++u) {
    const int i = b + t + u * kSliceThreads;
    v[u] = i < e ? l[i] : 0.f;
  }
  double s = 0.0, sf = 0.0;
  int nf = 0;
  float w1 = -1.f, w2 = -1.f;
  int i1 = INT_MAX, i2 = INT_MAX;
#pragma unroll
  for (int u = 0; u < kSlice / kSliceThreads; ++u) {
    const int i = b + t + u * kSliceThreads;
    if (i < e) {
      const float x = expf((v[u] - mx) * inv_t);
      w[i] = x;
      s += double(x);
      if (x >= floor_w) sf += double(x), ++nf;
      if (more_likely(x, i, w1, i1)) {
        w2 = w1, i2 = i1;
        w1 = x, i1 = i;
      } else if (more_likely(x, i, w2, i2)) {
        w2 = x, i2 = i;
      }
    }
  }
  s = wave_sum_d(s);
  sf = wave_sum_d(sf);
  for (int o = 32; o >= 1; o >>= 1) nf += __shfl_xor(nf, o);
  const float m2 = wave_max(w2);
  if ((t & 63) == 0) dred[t >> 6][0] = s, dred[t >> 6][1] = sf, ired[t >> 6] = nf, m2red[t >> 6] = m2;
  const size_t so = size_t(row) * a.slices + sl;
  if (a.lists) {
    // the thread's summary: the gather of candidates at or above a threshold reads it instead of the row
    const size_t th = so * kSliceThreads + size_t(t);
    a.tmax[th] = w1;
    a.tsec[th] = w2;
    a.tu[th] = uint8_t(i1 == INT_MAX ? 0 : (i1 - b - t) / kSliceThreads);
    // the threads' first pairs in candidate order: each wave's 64 in registers, then merged
    unsigned long long kq = pair_key(w1, i1);
    wave_sort64(kq);
    ck[t] = kq;
    merge_runs<kSliceThreads>(ck, tk, kSliceThreads, 64);
    if (t < kSliceTop) {
      a.sw[so * kSliceTop + t] = key_w(ck[t]);
      a.si[so * kSliceTop + t] = key_id(ck[t]);
    }
  } else {
    __syncthreads();
  }
  if (t == 0) {
    double ts = 0.0, tf = 0.0;
    int tn = 0;
    float tm2 = -1.f;
    for (int q = 0; q < kSliceThreads / 64; ++q)
      ts += dred[q][0], tf += dred[q][1], tn += ired[q], tm2 = fmaxf(tm2, m2red[q]);
    a.ssum[so] = ts;
    a.sfl[so] = tf;
    a.snfl[so] = tn;
    a.sm2[so] = tm2;
  }
}

// One work-group per row: the slices' sums in order, then the walk (index order, no filter) or the filters over
// the candidates in order (sampler.cpp:44-94).
__global__ void __launch_bounds__(kSampleThreads) sample_pick_kernel(const SampleArgs a) {
  __shared__ double red[kSampleThreads / 64 + 4];   // >= 20
  __shared__ uint32_t ured[kSampleThreads / 64 + 1];
  // the whole-row sort's digit counts, or the merges' scratch keys
  __shared__ __align__(16) uint32_t hist[16 * kSampleThreads];
  static_assert(2 * kCand <= 16 * kSampleThreads, "scratch keys in hist");
  __shared__ unsigned long long ck[kCand];   // candidates as pair keys
  unsigned long long* tk = reinterpret_cast<unsigned long long*>(hist);
  __shared__ unsigned long long selh[256];
  __shared__ int sel, ccount, slices_ok, nread;
  __shared__ unsigned long long above_s;
  __shared__ double base_s;
  const int row = int(blockIdx.x), t = int(threadIdx.x), n = a.n, S = a.slices;
  const float* w = a.w + size_t(row) * size_t(n);
  const size_t so = size_t(row) * S;
  const float floor_w = a.min_p * 1.0f;

  // totals over the row: slice by slice, in order; the slices' figures (written on other XCDs) go through LDS in
  // chunks of 1024, loaded in parallel, and one thread adds them in order
  double* lsum = reinterpret_cast<double*>(hist);
  double* lfl = lsum + kSampleThreads;
  int* lnf = reinterpret_cast<int*>(lfl + kSampleThreads);
  {
    double tot = 0.0, tf = 0.0;
    int nf = 0;
    for (int b = 0; b < S; b += kSampleThreads) {
      if (b + t < S) {
        lsum[t] = a.ssum[so + b + t];
        lfl[t] = a.sfl[so + b + t];
        lnf[t] = a.snfl[so + b + t];
      }
      __syncthreads();
      if (t == 0) {
        const int m = min(kSampleThreads, S - b);
#pragma unroll 8
        for (int i = 0; i < m; ++i) tot += lsum[i], tf += lfl[i], nf += lnf[i];
      }
      __syncthreads();
    }
    if (t == 0) {
      red[0] = tot;
      red[1] = tf;
      ccount = nf;
    }
  }
  __syncthreads();
  double total = red[0];
  const double t_floor = red[1];
  const int n_floor = ccount;
  __syncthreads();

  const bool topk = a.top_k > 0 && a.top_k < n;
  if (!topk && a.top_p >= 1.f && a.min_p <= 0.f) {   // no filter: the candidates in index order
    const double r = a.u[row] * total;
    if (t == 0) {   // the slice where the running sum passes r, and the running sum before it (8 sums read at once)
      double c = 0.0;
      int q = 0;
      bool done = false;
      for (int q0 = 0; q0 < S && !done; q0 += 8) {
        double v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = q0 + i < S ? (S <= kSampleThreads ? lsum[q0 + i] : a.ssum[so + q0 + i]) : 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (!done) {
            if (q0 + i >= S - 1 || c + v[i] > r) {
              q = q0 + i;
              done = true;
            } else {
              c += v[i];
            }
          }
        }
      }
      sel = q;
      base_s = c;
    }
    __syncthreads();
    const int q = sel;
    const double c0 = base_s;
    const int b = q * kSlice, len = min(n, b + kSlice) - b;
    double at;
    const int i = first_crossing([&](int j) { return w[b + j]; }, len, r, true, red, &sel, &at, c0);
    if (t == 0) a.out[row] = b + (i < len ? i : len - 1);   // past every crossing: the slice's (the row's) last
    return;
  }

  // tau, a weight that the kept prefix cannot go below, from the union of the slices' lists (S * 64 pairs): for
  // top_k up to 64 the union's top_k-th pair, from merges that keep each pair of runs' first 64; otherwise
  // union_select's bucket edge where the union's count reaches top_k, or where its mass reaches total * top_p *
  // (1 + 1e-6); the floor for min_p (the larger of the two with top_p). The union is a subset of the row, so the row
  // holds at least as much at or above tau.
  const int U = S * kSliceTop;
  const float* uw = a.sw + so * kSliceTop;
  const int* ui = a.si + so * kSliceTop;
  const bool top_only = topk && a.top_k <= kSliceTop && U <= kCand;
  const float last_p = t < S ? uw[size_t(t) * kSliceTop + kSliceTop - 1] : 0.f;
  const float m2_p = t < S ? a.sm2[so + t] : 0.f;
  int nc = INT_MAX;        // candidates in ck (INT_MAX: none yet)
  bool in_order = false;   // in candidate order already
  float tau = -1.f;
  if (top_only) {
    int n2 = 1;
    while (n2 < U) n2 <<= 1;
    for (int q = t; q < n2; q += kSampleThreads) ck[q] = q < U ? pair_key(uw[q], ui[q]) : kPadKey;
    // every slice's list (and the padding) is a run of kSliceTop in candidate order; top_k up to kSliceTop needs
    // only the union's first kSliceTop (the filters never look past the first top_k candidates)
    merge_top<kSampleThreads>(ck, tk, n2 / kSliceTop, kSliceTop);
    const float wk = key_w(ck[a.top_k - 1]);
    tau = wk >= 0.f ? wk : -1.f;
  } else if (topk) {
    tau = a.top_k <= U ? union_select(uw, U, false, double(a.top_k), selh, &sel, &above_s) : -1.f;
  } else {
    if (a.top_p < 1.f) {
      const double target = total * double(a.top_p) * (1.0 + 1e-6);   // the union's mass is at most U
      tau = target < double(U) ? union_select(uw, U, true, target, selh, &sel, &above_s) : -1.f;
    }
    if (a.min_p > 0.f) tau = fmaxf(tau, floor_w);   // min_p keeps nothing below its floor
  }
  // every weight >= tau is a listed thread maximum when, in every slice, the 64th listed maximum and every thread's
  // second most likely lie below tau (the first 1024 slices' figures were loaded before tau was known)
  if (t == 0) slices_ok = 1;
  __syncthreads();
  if (tau >= 0.f)
    for (int q = t; q < S; q += kSampleThreads) {
      const float last = q == t ? last_p : uw[size_t(q) * kSliceTop + kSliceTop - 1];
      const float m2 = q == t ? m2_p : a.sm2[so + q];
      if (!(last < tau) || !(m2 < tau)) atomicAnd(&slices_ok, 0);   // ties or runs at tau may continue past the lists
    }
  __syncthreads();
  if (tau >= 0.f && slices_ok && top_only) {   // the union's prefix at or above tau, already in order
    if (t == 0) sel = kSliceTop;
    __syncthreads();
    for (int q = t; q < kSliceTop; q += kSampleThreads)
      if (!(key_w(ck[q]) >= tau)) atomicMin(&sel, q);
    __syncthreads();
    nc = sel;
    in_order = true;
    __syncthreads();
  } else if (tau >= 0.f && slices_ok && U <= kCand) {   // the union's pairs at or above tau (sorted next)
    constexpr int PT = kCand / kSampleThreads;
    float x[PT];
    int xi[PT];
    int c = 0;
#pragma unroll
    for (int r = 0; r < PT; ++r) {
      const int e = PT * t + r;
      x[r] = e < U ? uw[e] : -1.f;
      xi[r] = e < U ? ui[e] : 0;
      c += x[r] >= tau ? 1 : 0;
    }
    uint32_t tot;
    int at = int(block_exclusive<uint32_t>(uint32_t(c), ured, &tot));
#pragma unroll
    for (int r = 0; r < PT; ++r)
      if (x[r] >= tau) ck[at++] = pair_key(x[r], xi[r]);
    nc = int(tot);
  }
  const uint32_t* ksrc = nullptr;
  const int* isrc = nullptr;
  int L;   // candidates available in order
  if (in_order) {
    L = nc;
  } else {
    // gather every weight >= tau from the row (order-free, then sorted) unless the union supplied them, or sort the
    // whole row
    if (t == 0) ccount = 0;
    __syncthreads();
    if (nc == INT_MAX && tau >= 0.f) {
      // from the slices' thread summaries, 16 slice threads a thread with every load in flight (they were written on
      // other XCDs): a slice thread whose second most likely lies below tau holds at most its first, at b + t + 256 u;
      // one whose second reaches tau is listed, and its weights are read from the row next. A wave takes places for
      // the first kind with one atomic, each hit of the second kind one (the order is free: the pairs are sorted next).
      constexpr int PT = 16;
      constexpr int kReadCap = kCand / 2;   // slice threads to read from the row (each holds >= 2 candidates)
      int* rlist = reinterpret_cast<int*>(hist);
      if (t == 0) nread = 0;
      __syncthreads();
      const int lane = t & 63;
      const int nth = S * kSliceThreads;   // a multiple of PT
      const size_t tb = so * kSliceThreads;
      for (int j0 = 0; j0 < nth; j0 += PT * kSampleThreads) {   // the same rounds in every thread
        const int j = j0 + PT * t;
        float fm[PT], fs[PT];
        uint8_t fu[PT];
        if (j < nth) {
#pragma unroll
          for (int q = 0; q < PT / 4; ++q) {
            const float4 m4 = *reinterpret_cast<const float4*>(a.tmax + tb + j + 4 * q);
            const float4 s4 = *reinterpret_cast<const float4*>(a.tsec + tb + j + 4 * q);
            fm[4 * q] = m4.x, fm[4 * q + 1] = m4.y, fm[4 * q + 2] = m4.z, fm[4 * q + 3] = m4.w;
            fs[4 * q] = s4.x, fs[4 * q + 1] = s4.y, fs[4 * q + 2] = s4.z, fs[4 * q + 3] = s4.w;
          }
          const uint4 u4 = *reinterpret_cast<const uint4*>(a.tu + tb + j);
          const uint32_t uw4[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
          for (int q = 0; q < PT; ++q) fu[q] = uint8_t(uw4[q >> 2] >> (8 * (q & 3)));
        } else {
#pragma unroll
          for (int q = 0; q < PT; ++q) fm[q] = fs[q] = -1.f, fu[q] = 0;
        }
        int c = 0;
#pragma unroll
        for (int q = 0; q < PT; ++q) c += fs[q] < tau && fm[q] >= tau ? 1 : 0;
        int incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o);
          if (lane >= o) incl += y;
        }
        const int wtot = __shfl(incl, 63);
        int wb = 0;
        if (lane == 0 && wtot > 0) wb = atomicAdd(&ccount, wtot);
        int pos = __shfl(wb, 0) + incl - c;
#pragma unroll
        for (int q = 0; q < PT; ++q) {
          const int jj = j + q, sl = jj / kSliceThreads, tt = jj % kSliceThreads;
          if (fs[q] < tau && fm[q] >= tau) {
            if (pos < kCand) ck[pos] = pair_key(fm[q], sl * kSlice + tt + kSliceThreads * int(fu[q]));
            ++pos;
          } else if (fs[q] >= tau) {
            const int at = atomicAdd(&nread, 1);
            if (at < kReadCap) rlist[at] = jj;
          }
        }
      }
      // the listed slice threads' weights from the row, 8 threads to each, all loads at once; more than kReadCap of
      // them hold more than kCand candidates, which the whole-row sort takes
      __syncthreads();
      const int nr = min(nread, kReadCap);
      constexpr int PU = kSlice / kSliceThreads;
      for (int e = t; e < nr * PU; e += kSampleThreads) {
        const int jj = rlist[e / PU], u = e % PU;
        const int i = (jj / kSliceThreads) * kSlice + jj % kSliceThreads + u * kSliceThreads;
        const float x = i < n ? w[i] : -1.f;
        if (x >= tau) {
          const int at = atomicAdd(&ccount, 1);
          if (at < kCand) ck[at] = pair_key(x, i);
        }
      }
      if (t == 0 && nread > kReadCap) atomicMax(&ccount, kCand + 1);
    }
    __syncthreads();
    if (nc == INT_MAX) nc = tau >= 0.f ? ccount : INT_MAX;
    __syncthreads();
    if (nc <= kCand) {
      int n2 = 1;
      while (n2 < nc) n2 <<= 1;
      for (int q = nc + t; q < n2; q += kSampleThreads) ck[q] = kPadKey;
      sort_pairs<kSampleThreads>(ck, tk, n2);
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
  }
  auto sw = [&](int j) { return ksrc ? __uint_as_float(~ksrc[j]) : key_w(ck[j]); };
  auto sidx = [&](int j) { return ksrc ? isrc[j] : key_id(ck[j]); };

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
    } else {   // every weight >= floor: counted over the row with the weights
      k = n_floor;
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

namespace {
struct SampleScratch {
  size_t w, smax, sbest, sbi, ssum, sfl, snfl, sw, si, sm2, tmax, tsec, tu, keys, idx, total;
};
SampleScratch scratch_layout(int rows, int n) {
  const size_t S = size_t((n + kSlice - 1) / kSlice), R = size_t(rows), N = size_t(n);
  SampleScratch o{};
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t p = at;
    at += (bytes + 255) / 256 * 256;
    return p;
  };
  o.ssum = take(R * S * 8);
  o.sfl = take(R * S * 8);
  o.w = take(R * N * 4);
  o.smax = take(R * S * 4);
  o.sbest = take(R * S * 4);
  o.sbi = take(R * S * 4);
  o.snfl = take(R * S * 4);
  o.sw = take(R * S * kSliceTop * 4);
  o.si = take(R * S * kSliceTop * 4);
  o.sm2 = take(R * S * 4);
  o.tmax = take(R * S * kSliceThreads * 4);
  o.tsec = take(R * S * kSliceThreads * 4);
  o.tu = take(R * S * kSliceThreads);
  o.keys = take(R * 2 * N * 4);
  o.idx = take(R * 2 * N * 4);
  o.total = at;
  return o;
}

SampleArgs sample_args(const float* logits, int rows, int n, void* scratch, int* out) {
  const SampleScratch o = scratch_layout(rows, n);
  char* base = static_cast<char*>(scratch);
  SampleArgs a{};
  a.logits = logits;
  a.n = n;
  a.slices = (n + kSlice - 1) / kSlice;
  a.w = reinterpret_cast<float*>(base + o.w);
  a.smax = reinterpret_cast<float*>(base + o.smax);
  a.sbest = reinterpret_cast<float*>(base + o.sbest);
  a.sbi = reinterpret_cast<int*>(base + o.sbi);
  a.ssum = reinterpret_cast<double*>(base + o.ssum);
  a.sfl = reinterpret_cast<double*>(base + o.sfl);
  a.snfl = reinterpret_cast<int*>(base + o.snfl);
  a.sw = reinterpret_cast<float*>(base + o.sw);
  a.si = reinterpret_cast<int*>(base + o.si);
  a.sm2 = reinterpret_cast<float*>(base + o.sm2);
  a.tmax = reinterpret_cast<float*>(base + o.tmax);
  a.tsec = reinterpret_cast<float*>(base + o.tsec);
  a.tu = reinterpret_cast<uint8_t*>(base + o.tu);
  a.keys = reinterpret_cast<uint32_t*>(base + o.keys);
  a.idx = reinterpret_cast<int*>(base + o.idx);
  a.out = out;
  return a;
}
}  // namespace

size_t sample_scratch_bytes(int rows, int n) { return scratch_layout(rows, n).total; }

std::string launch_sample(const float* logits, int rows, int n, float temperature, float top_p, int top_k,
                          float min_p, const double* u, int* out, void* scratch, hipStream_t stream) {
  XTG_CHECK(rows >= 1 && rows <= kMaxSampleRows, "sample: %d rows (1..%d)", rows, kMaxSampleRows);
  XTG_CHECK(n >= 1, "sample: %d logits", n);
  XTG_CHECK(temperature > 0.f, "sample: temperature %g (greedy decoding is argmax)", double(temperature));
  SampleArgs a = sample_args(logits, rows, n, scratch, out);
  a.temperature = temperature;
  a.top_p = top_p;
  a.min_p = min_p;
  a.top_k = top_k;
  a.lists = (top_k > 0 && top_k < n) || top_p < 1.f || min_p > 0.f ? 1 : 0;
  for (int r = 0; r < rows; ++r) {
    XTG_CHECK(u[r] >= 0.0 && u[r] < 1.0, "sample: draw %g outside [0, 1)", u[r]);
    a.u[r] = u[r];
  }
  const dim3 sg{unsigned(a.slices), unsigned(rows)};
  hipLaunchKernelGGL(slice_max_kernel, sg, dim3(kSliceThreads), 0, stream, a);
  hipLaunchKernelGGL(slice_weights_kernel, sg, dim3(kSliceThreads), 0, stream, a);
  hipLaunchKernelGGL(sample_pick_kernel, dim3(unsigned(rows)), dim3(kSampleThreads), 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return "sample_pick_kernel";
}

std::string launch_argmax_slices(const float* logits, int rows, int n, int* out, void* scratch, hipStream_t stream) {
  XTG_CHECK(rows >= 1 && rows <= kMaxSampleRows && n >= 1, "argmax: %d rows of %d", rows, n);
  const SampleArgs a = sample_args(logits, rows, n, scratch, out);
  hipLaunchKernelGGL(slice_max_kernel, dim3(unsigned(a.slices), unsigned(rows)), dim3(kSliceThreads), 0, stream, a);
  hipLaunchKernelGGL(argmax_pick_kernel, dim3(unsigned(rows)), dim3(64), 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return "argmax_pick_kernel";
}

}  // namespace xtg::hip
