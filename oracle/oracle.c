/* CPU oracle: plain-C restatement of the reference engine's CPU kernels for the decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY -- see oracle.h. Built with the reference build's arithmetic flags
 * (-O3 -march=x86-64-v3 -fopenmp-simd, GNU dialect so FP contraction is on), so the FP32 summation structure
 * follows the reference's loops. Citations are reference paths.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------------ formats */

float xo_bf16_to_f32(uint16_t h) {
  /* engine/include/xtg/fp.h:10-15 */
  uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t xo_f32_to_bf16(float f) {
  /* engine/include/xtg/fp.h:18-24: round to nearest even, a NaN stays a (quiet) NaN */
  uint32_t bits;
  memcpy(&bits, &f, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

static float g_e4m3[256];
static int g_e4m3_ready = 0;

static void e4m3_init(void) {
  /* engine/src/fp.cpp:12-28: bias 7, subnormal step 2^-9, 0x7f / 0xff NaN, no infinities */
  if (g_e4m3_ready) return;
  for (int b = 0; b < 256; ++b) {
    int e = (b >> 3) & 15, m = b & 7;
    float mag;
    if ((b & 0x7f) == 0x7f)
      mag = NAN;
    else if (e == 0)
      mag = (float)m * ldexpf(1.f, -9);
    else
      mag = (1.f + (float)m / 8.f) * ldexpf(1.f, e - 7);
    g_e4m3[b] = (b & 0x80) ? -mag : mag;
  }
  g_e4m3_ready = 1;
}

__attribute__((constructor)) static void oracle_init(void) { e4m3_init(); }

float xo_e4m3_to_f32(uint8_t b) { return g_e4m3[b]; }

uint8_t xo_f32_to_e4m3(float f) {
  /* engine/src/fp.cpp:30-49: the largest code not above |f| by binary search, then round to nearest even;
   * |f| >= 448 saturates to 0x7e */
  uint8_t sign = signbit(f) ? 0x80 : 0;
  if (isnan(f)) return (uint8_t)(sign | 0x7f);
  float a = fabsf(f);
  if (a >= 448.f) return (uint8_t)(sign | 0x7e);
  int lo = 0, hi = 0x7e;
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if (g_e4m3[mid] <= a)
      lo = mid;
    else
      hi = mid - 1;
  }
  if (lo < 0x7e) {
    float d0 = a - g_e4m3[lo], d1 = g_e4m3[lo + 1] - a;
    if (d1 < d0 || (d1 == d0 && (lo & 1))) ++lo;
  }
  return (uint8_t)(sign | lo);
}

uint8_t xo_e4m3_bits(float x) {
  /* engine/src/kv.cpp:19-40: below 2^-6 count subnormal steps of 2^-9 (ties to even); above, round the FP32
   * mantissa to 3 bits (ties to even) and rebias, capped at 0x7e */
  uint32_t bits;
  memcpy(&bits, &x, 4);
  uint32_t sign = (bits >> 24) & 0x80u, a = bits & 0x7fffffffu, code;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (a < 0x3c800000u) {
    float t;
    memcpy(&t, &a, 4);
    t *= 512.f;
    float lo = floorf(t);
    uint32_t steps = (uint32_t)lo;
    float half = t - lo;
    steps += (half > 0.5f) || (half == 0.5f && (steps & 1u));
    code = steps;
  } else {
    uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    code = ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
    if (code > 0x7eu) code = 0x7eu;
  }
  return (uint8_t)(sign | code);
}

/* engine/include/xtg/fp.h:37-39 */
static const float kE2m1[16] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f,
                                -0.f, -0.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
float xo_e2m1(int code) { return kE2m1[code & 15]; }

/* ------------------------------------------------------------------------------------------------ NVFP4 */

void xo_nvfp4_row(const xo_nvfp4* w, int n, float* out) {
  /* engine/src/kernels.cpp:34-45: the scale and the tensor scale are folded into each decoded weight */
  const uint8_t* c = w->codes + (size_t)n * (size_t)(w->k / 2);
  const uint8_t* s = w->scales + (size_t)n * (size_t)(w->k / 16);
  for (int g = 0; g < w->k / 16; ++g) {
    float sc = g_e4m3[s[g]] * w->global;
    for (int j = 0; j < 8; ++j) {
      uint8_t b = c[g * 8 + j];
      out[g * 16 + 2 * j] = kE2m1[b & 15] * sc;
      out[g * 16 + 2 * j + 1] = kE2m1[b >> 4] * sc;
    }
  }
}

static float dot_nvfp4(const xo_nvfp4* w, int n, const float* x) {
  /* engine/src/kernels.cpp:48-60: per 16-input group the E2M1 products are summed in FP32, then scaled by the
   * group's E4M3 value; the tensor scale multiplies the total */
  const uint8_t* c = w->codes + (size_t)n * (size_t)(w->k / 2);
  const uint8_t* s = w->scales + (size_t)n * (size_t)(w->k / 16);
  float acc = 0.f;
  for (int g = 0; g < w->k / 16; ++g) {
    const uint8_t* cg = c + g * 8;
    const float* xg = x + g * 16;
    float part = 0.f;
    for (int j = 0; j < 8; ++j) part += kE2m1[cg[j] & 15] * xg[2 * j] + kE2m1[cg[j] >> 4] * xg[2 * j + 1];
    acc += part * g_e4m3[s[g]];
  }
  return acc * w->global;
}

/* engine/src/kernels.cpp:62-67 (a separate translation unit in the reference, hence not inlined here) */
__attribute__((noinline)) static float dot_f32(const float* a, const float* b, int k) {
  float s = 0.f;
#pragma omp simd reduction(+ : s)
  for (int j = 0; j < k; ++j) s += a[j] * b[j];
  return s;
}

int xo_matmul_nvfp4(const xo_nvfp4* ws, int n_w, const float* x, int m, float* const* ys, int threads) {
  /* engine/src/kernels.cpp:84-138. Several weights reading the same x form one list of rows (RowMap :69-82);
   * which rows a thread takes changes nothing in the results, so the rows are walked weight by weight. */
  if (n_w <= 0) return -1;
  const int k = ws[0].k;
  for (int i = 0; i < n_w; ++i)
    if (ws[i].k != k || k % 16 != 0) return -1;
  if (threads < 1) threads = 1;
  for (int wi = 0; wi < n_w; ++wi) {
    const xo_nvfp4* w = &ws[wi];
    float* y = ys[wi];
    if (m <= 2) {
      /* decode branch (:90-114): one dot_nvfp4 per (input row, output row) */
#pragma omp parallel for num_threads(threads) schedule(static)
      for (int n = 0; n < w->n_out; ++n)
        for (int i = 0; i < m; ++i) y[(size_t)i * (size_t)w->n_out + (size_t)n] = dot_nvfp4(w, n, x + (size_t)i * (size_t)k);
    } else {
      /* prefill branch (:116-137): the weight row decoded to FP32 (scales folded in), then dot_f32 per input row */
#pragma omp parallel num_threads(threads)
      {
        float* wrow = (float*)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
        for (int n = 0; n < w->n_out; ++n) {
          xo_nvfp4_row(w, n, wrow);
          for (int i = 0; i < m; ++i)
            y[(size_t)i * (size_t)w->n_out + (size_t)n] = dot_f32(wrow, x + (size_t)i * (size_t)k, k);
        }
        free(wrow);
      }
    }
  }
  return 0;
}

int xo_matmul_bf16(const uint16_t* w, int n_out, int k, const float* x, int m, float* y, int threads) {
  /* engine/src/kernels.cpp:140-155: each weight row converted to FP32, then dot_f32 with every input row */
  if (n_out <= 0 || k <= 0 || m <= 0) return -1;
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
  {
    float* wrow = (float*)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
    for (int n = 0; n < n_out; ++n) {
      const uint16_t* r = w + (size_t)n * (size_t)k;
      for (int j = 0; j < k; ++j) wrow[j] = xo_bf16_to_f32(r[j]);
      for (int i = 0; i < m; ++i) y[(size_t)i * (size_t)n_out + (size_t)n] = dot_f32(wrow, x + (size_t)i * (size_t)k, k);
    }
    free(wrow);
  }
  return 0;
}

/* --------------------------------------------------------------------------------------------- row kernels */

void xo_bf16_row(const uint16_t* table, int64_t row, int width, float* out) {
  /* engine/src/kernels.cpp:157-160 */
  const uint16_t* r = table + row * width;
  for (int j = 0; j < width; ++j) out[j] = xo_bf16_to_f32(r[j]);
}

__attribute__((noinline)) static float inv_norm(const float* x, int w) {
  /* engine/src/kernels.cpp:162-167 */
  float s = 0.f;
#pragma omp simd reduction(+ : s)
  for (int j = 0; j < w; ++j) s += x[j] * x[j];
  return 1.f / sqrtf(s + 1e-6f);
}

void xo_justnorm(float* x, int rows, int width) {
  /* engine/src/kernels.cpp:169-175 */
  for (int r = 0; r < rows; ++r) {
    float* v = x + (size_t)r * (size_t)width;
    float f = inv_norm(v, width);
    for (int j = 0; j < width; ++j) v[j] *= f;
  }
}

void xo_slerp_residual(float* a, const float* b, const float* lr, int rows, int width) {
  /* engine/src/kernels.cpp:177-189 */
  for (int r = 0; r < rows; ++r) {
    float* va = a + (size_t)r * (size_t)width;
    const float* vb = b + (size_t)r * (size_t)width;
    float fa = inv_norm(va, width), fb = inv_norm(vb, width);
    for (int j = 0; j < width; ++j) {
      float ya = va[j] * fa, yb = vb[j] * fb;
      va[j] = ya + lr[j] * (yb - ya);
    }
    float f = inv_norm(va, width);
    for (int j = 0; j < width; ++j) va[j] *= f;
  }
}

static void inv_freq(float theta, int d, float* f) {
  /* engine/src/kernels.cpp:191-201: 1 / theta^(2i/d) in FP32 */
  for (int i = 0; i < d / 2; ++i) f[i] = 1.f / powf(theta, (float)(2 * i) / (float)d);
}

void xo_rope(float* x, int rows, int heads, int head_dim, int64_t pos0, float theta) {
  /* engine/src/kernels.cpp:203-223: NeoX half split; angle = FP32(pos) * inv_freq in FP32 */
  const int half = head_dim / 2;
  float* f = (float*)malloc(sizeof(float) * (size_t)half * 3);
  float* c = f + half;
  float* s = c + half;
  inv_freq(theta, head_dim, f);
  for (int r = 0; r < rows; ++r) {
    float pos = (float)(pos0 + r);
    for (int i = 0; i < half; ++i) {
      float a = pos * f[i];
      c[i] = cosf(a);
      s[i] = sinf(a);
    }
    for (int h = 0; h < heads; ++h) {
      float* v = x + ((size_t)r * (size_t)heads + (size_t)h) * (size_t)head_dim;
      for (int i = 0; i < half; ++i) {
        float x1 = v[i], x2 = v[i + half];
        v[i] = x1 * c[i] - x2 * s[i];
        v[i + half] = x2 * c[i] + x1 * s[i];
      }
    }
  }
  free(f);
}

void xo_rope_table(float* cs, int m, int head_dim, int64_t pos0, float theta) {
  /* packs/dory/dory.cpp:1159-1171: the same FP32 angles as rope(), laid out [cos rows][sin rows] */
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    float inv = 1.f / powf(theta, (float)(2 * i) / (float)head_dim);
    for (int r = 0; r < m; ++r) {
      float a = (float)(pos0 + r) * inv;
      cs[(size_t)r * (size_t)half + (size_t)i] = cosf(a);
      cs[(size_t)(m + r) * (size_t)half + (size_t)i] = sinf(a);
    }
  }
}

void xo_swiglu_scaled(float* g, const float* u, const float* sg, const float* su, int rows, int w) {
  /* engine/src/kernels.cpp:225-234 */
  for (int r = 0; r < rows; ++r) {
    float* gr = g + (size_t)r * (size_t)w;
    const float* ur = u + (size_t)r * (size_t)w;
    for (int j = 0; j < w; ++j) {
      float z = gr[j] * sg[j];
      gr[j] = z / (1.f + expf(-z)) * (ur[j] * su[j]);
    }
  }
}

void xo_gate_norm(float* att, const float* gate, const float* gs, int rows, int width) {
  /* packs/dory/dory.cpp:510-515: sigmoid output gate, then a norm over all heads */
  for (int r = 0; r < rows; ++r) {
    float* ar = att + (size_t)r * (size_t)width;
    const float* gr = gate + (size_t)r * (size_t)width;
    for (int j = 0; j < width; ++j) ar[j] *= 1.f / (1.f + expf(-gr[j] * gs[j]));
  }
  xo_justnorm(att, rows, width);
}

int xo_argmax(const float* x, int n) {
  /* engine/src/sampler.cpp:8-13: the first index whose value no later value exceeds; a NaN never compares
     greater (and a NaN at 0 is never displaced) */
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

/* engine/src/sampler.cpp:26-28: larger weight first, then smaller index (a strict total order on candidates) */
typedef struct {
  float w;
  int i;
} xo_cand;
static int xo_more_likely_cmp(const void* pa, const void* pb) {
  const xo_cand* a = (const xo_cand*)pa;
  const xo_cand* b = (const xo_cand*)pb;
  if (a->w > b->w || (a->w == b->w && a->i < b->i)) return -1;
  if (b->w > a->w || (a->w == b->w && b->i < a->i)) return 1;
  return 0;
}

static void xo_margin(double* m, double x, double boundary, double total) {
  const double d = fabs(x - boundary) / (total > 0.0 ? total : 1.0);
  if (d < *m) *m = d;
}

int xo_sample(const float* logits, int n, float temperature, float top_p, int top_k, float min_p, double u,
              double* margin) {
  /* engine/src/sampler.cpp:40-94 with r = u * total (uniform_real_distribution<double>(0, total) scales the
     generator's generate_canonical draw u by the total). The candidates are fully sorted whenever a filter
     applies: the reference's partial sorts order the same leading candidates, which are all its filters read
     wherever its result is defined. margin (optional): the smallest distance, relative to the total, between r
     (or the top_p target) and a running sum next to the chosen position. */
  double mg = INFINITY;
  if (temperature <= 0.f) {
    if (margin) *margin = mg;
    return xo_argmax(logits, n);
  }
  float mx = logits[0];
  for (int i = 1; i < n; ++i) mx = mx < logits[i] ? logits[i] : mx; /* std::max(mx, logits[i]) */
  const float inv_t = 1.f / temperature;
  xo_cand* c = (xo_cand*)malloc(sizeof(xo_cand) * (size_t)n);
  double total = 0.0;
  for (int i = 0; i < n; ++i) {
    const float w = expf((logits[i] - mx) * inv_t);
    c[i].w = w;
    c[i].i = i;
    total += w;
  }
  int keep = n;
  if (top_k > 0 && top_k < n) {
    qsort(c, (size_t)n, sizeof(xo_cand), xo_more_likely_cmp);
    keep = top_k;
    total = 0.0;
    for (int i = 0; i < keep; ++i) total += c[i].w;
  } else if (top_p < 1.f || min_p > 0.f) {
    qsort(c, (size_t)n, sizeof(xo_cand), xo_more_likely_cmp);
  }
  if (min_p > 0.f) {
    const float floor_w = min_p * c[0].w;
    int k = 0;
    double t = 0.0;
    while (k < keep && c[k].w >= floor_w) t += c[k++].w;
    keep = k > 1 ? k : 1;
    total = k ? t : (double)c[0].w;
  }
  if (top_p < 1.f) {
    const double target = total * (double)top_p;
    double cum = 0.0;
    int k = 0;
    while (k < keep) {
      const double before = cum;
      cum += c[k].w;
      ++k;
      if (cum >= target) {
        xo_margin(&mg, target, before, total);
        xo_margin(&mg, target, cum, total);
        break;
      }
    }
    keep = k > 1 ? k : 1;
    total = cum;
  }
  const double r = u * total;
  double cum = 0.0;
  int token = c[keep - 1].i;
  for (int i = 0; i < keep; ++i) {
    const double before = cum;
    cum += c[i].w;
    if (r < cum) {
      token = c[i].i;
      xo_margin(&mg, r, before, total);
      xo_margin(&mg, r, cum, total);
      break;
    }
  }
  free(c);
  if (margin) *margin = mg;
  return token;
}

void xo_add_norm(const float* a, const float* b, float* out, int rows, int width) {
  /* packs/dory/dory.cpp:532-541: loop entry x = justnorm(state + input); loop exit state = justnorm(x) */
  const size_t n = (size_t)rows * (size_t)width;
  for (size_t i = 0; i < n; ++i) out[i] = b ? a[i] + b[i] : a[i];
  xo_justnorm(out, rows, width);
}

void xo_qk_produce(float* q, float* k, int m, int heads, int kv_heads, int head_dim, int64_t pos0, float theta,
                   const float* qscale) {
  /* packs/dory/dory.cpp:482-490: RoPE on q and k, then justnorm per head, then q times the per-dimension
   * scale over all heads (qscale has heads * head_dim entries); k is not scaled */
  const int Q = heads * head_dim;
  xo_rope(q, m, heads, head_dim, pos0, theta);
  xo_rope(k, m, kv_heads, head_dim, pos0, theta);
  xo_justnorm(q, m * heads, head_dim);
  for (int r = 0; r < m; ++r) {
    float* qr = q + (size_t)r * (size_t)Q;
    for (int j = 0; j < Q; ++j) qr[j] *= qscale[j];
  }
  xo_justnorm(k, m * kv_heads, head_dim);
}

/* ---------------------------------------------------------------------------------------------- KV cache */

struct xo_kv {
  int kv_heads, head_dim;
  int64_t slots;
  int ring, dtype;
  size_t elem;
  uint8_t* k;
  uint8_t* v;
  float* ks;
  float* vs;
};

xo_kv* xo_kv_create(int kv_heads, int head_dim, int64_t slots, int ring, int dtype) {
  /* engine/src/kv.cpp:42-63: ring > 0 gives a ring of `ring` slots; storage [slots][kv_heads][head_dim] */
  xo_kv* c = (xo_kv*)calloc(1, sizeof(xo_kv));
  c->kv_heads = kv_heads;
  c->head_dim = head_dim;
  c->slots = ring > 0 ? ring : slots;
  c->ring = ring > 0;
  c->dtype = dtype;
  c->elem = dtype == XO_KV_FP8 ? 1 : 2;
  if (c->slots <= 0) {
    free(c);
    return NULL;
  }
  size_t n = (size_t)c->slots * (size_t)kv_heads * (size_t)head_dim;
  c->k = (uint8_t*)calloc(n, c->elem);
  c->v = (uint8_t*)calloc(n, c->elem);
  if (dtype == XO_KV_FP8) {
    c->ks = (float*)calloc((size_t)c->slots * (size_t)kv_heads, sizeof(float));
    c->vs = (float*)calloc((size_t)c->slots * (size_t)kv_heads, sizeof(float));
  }
  return c;
}

void xo_kv_free(xo_kv* c) {
  if (!c) return;
  free(c->k);
  free(c->v);
  free(c->ks);
  free(c->vs);
  free(c);
}

int64_t xo_kv_slots(const xo_kv* c) { return c->slots; }
const void* xo_kv_kdata(const xo_kv* c) { return c->k; }
const void* xo_kv_vdata(const xo_kv* c) { return c->v; }
const float* xo_kv_kscale(const xo_kv* c) { return c->ks; }
const float* xo_kv_vscale(const xo_kv* c) { return c->vs; }

int xo_kv_store(xo_kv* c, int64_t pos, int n, const float* k, const float* v) {
  /* engine/src/kv.cpp:75-112: a ring keeps the last `slots` rows of a long call; BF16 rows rounded to nearest
   * even; FP8 rows take a per-(position, head) scale amax / 448 and the kv.cpp rounding */
  int64_t first = pos;
  if (c->ring && n > c->slots) first = pos + n - c->slots;
  if (!c->ring && pos + n > c->slots) return -1;
  const size_t hd = (size_t)c->head_dim;
  for (int64_t p = first; p < pos + n; ++p) {
    int64_t slot = c->ring ? p % c->slots : p;
    for (int h = 0; h < c->kv_heads; ++h) {
      const float* src_k = k + ((size_t)(p - pos) * (size_t)c->kv_heads + (size_t)h) * hd;
      const float* src_v = v + ((size_t)(p - pos) * (size_t)c->kv_heads + (size_t)h) * hd;
      size_t idx = (size_t)slot * (size_t)c->kv_heads + (size_t)h;
      if (c->dtype == XO_KV_BF16) {
        uint16_t* dk = (uint16_t*)c->k + idx * hd;
        uint16_t* dv = (uint16_t*)c->v + idx * hd;
        for (size_t j = 0; j < hd; ++j) {
          dk[j] = xo_f32_to_bf16(src_k[j]);
          dv[j] = xo_f32_to_bf16(src_v[j]);
        }
      } else {
        float ak = 0.f, av = 0.f;
        for (size_t j = 0; j < hd; ++j) {
          ak = fmaxf(ak, fabsf(src_k[j]));
          av = fmaxf(av, fabsf(src_v[j]));
        }
        float sk = ak > 0.f ? ak / 448.f : 1.f, sv = av > 0.f ? av / 448.f : 1.f;
        float ik = 1.f / sk, iv = 1.f / sv;
        uint8_t* dk = c->k + idx * hd;
        uint8_t* dv = c->v + idx * hd;
        for (size_t j = 0; j < hd; ++j) {
          dk[j] = xo_e4m3_bits(src_k[j] * ik);
          dv[j] = xo_e4m3_bits(src_v[j] * iv);
        }
        c->ks[idx] = sk;
        c->vs[idx] = sv;
      }
    }
  }
  return 0;
}

void xo_kv_load(const xo_kv* c, int h, int64_t p0, int64_t p1, float* k, float* v) {
  /* engine/src/kv.cpp:114-138 */
  const size_t hd = (size_t)c->head_dim;
  for (int64_t p = p0; p < p1; ++p) {
    int64_t slot = c->ring ? p % c->slots : p;
    size_t idx = (size_t)slot * (size_t)c->kv_heads + (size_t)h;
    float* ok = k + (size_t)(p - p0) * hd;
    float* ov = v + (size_t)(p - p0) * hd;
    if (c->dtype == XO_KV_BF16) {
      const uint16_t* sk = (const uint16_t*)c->k + idx * hd;
      const uint16_t* sv = (const uint16_t*)c->v + idx * hd;
      for (size_t j = 0; j < hd; ++j) {
        ok[j] = xo_bf16_to_f32(sk[j]);
        ov[j] = xo_bf16_to_f32(sv[j]);
      }
    } else {
      const uint8_t* sk = c->k + idx * hd;
      const uint8_t* sv = c->v + idx * hd;
      float fk = c->ks[idx], fv = c->vs[idx];
      for (size_t j = 0; j < hd; ++j) {
        ok[j] = g_e4m3[sk[j]] * fk;
        ov[j] = g_e4m3[sv[j]] * fv;
      }
    }
  }
}

/* ----------------------------------------------------------------------------------------------- attention */

enum { kRows = 8, kTile = 64, kMaxGroup = 8 };   /* engine/src/kv.cpp:154-157 */

static int64_t lo_of(const xo_attn_args* a, int64_t t) {
  /* engine/src/kv.cpp:170: window > 0 -> keys t - window + 1 .. t */
  if (a->window <= 0) return 0;
  int64_t lo = t - a->window + 1;
  return lo > 0 ? lo : 0;
}

int xo_attention(const xo_attn_args* a, int pool_size, int threads) {
  /* engine/src/kv.cpp:166-286: tasks = kv_heads x blocks of 8 query rows x key splits; each task loads tiles of
   * 64 keys (cached positions from the cache, then this call's own keys in FP32), online softmax in FP32 per
   * (row, q head); splits are combined by their max / sum / accumulator */
  const int group = a->heads / a->kv_heads, d = a->head_dim;
  if (group * a->kv_heads != a->heads || group > kMaxGroup) return -1;
  if (threads < 1) threads = 1;
  const int64_t k_lo = lo_of(a, a->pos0), k_hi = a->pos0 + a->n_q;
  const int64_t span = k_hi - k_lo;
  const int qblocks = (a->n_q + kRows - 1) / kRows;
  int splits = 1;
  if (a->n_q <= 4 && span > 2 * kTile) {
    int64_t want = 2 * pool_size / a->kv_heads;
    if (want < 1) want = 1;
    int64_t cap = (span + 1023) / 1024;
    splits = (int)(want < cap ? want : cap);
  }
  if (splits < 1) splits = 1;
  const int64_t tasks = (int64_t)a->kv_heads * qblocks * splits;
  const size_t acc_per_task = (size_t)kRows * (size_t)group * (size_t)d;
  float* part_m = splits > 1 ? (float*)malloc(sizeof(float) * (size_t)tasks * kRows * kMaxGroup) : NULL;
  float* part_l = splits > 1 ? (float*)malloc(sizeof(float) * (size_t)tasks * kRows * kMaxGroup) : NULL;
  float* accs = splits > 1 ? (float*)malloc(sizeof(float) * (size_t)tasks * acc_per_task) : NULL;
  const float neg_inf = -INFINITY;

#pragma omp parallel num_threads(threads)
  {
    float* kt = (float*)malloc(sizeof(float) * (size_t)kTile * (size_t)d);
    float* vt = (float*)malloc(sizeof(float) * (size_t)kTile * (size_t)d);
    float* acc = (float*)malloc(sizeof(float) * acc_per_task);
    float sc[kTile];
    float st_m[kRows][kMaxGroup], st_l[kRows][kMaxGroup];
#pragma omp for schedule(dynamic, 1)
    for (int64_t task = 0; task < tasks; ++task) {
      int s = (int)(task % splits);
      int qb = (int)((task / splits) % qblocks);
      int h = (int)(task / ((int64_t)splits * qblocks));
      int i0 = qb * kRows, i1 = a->n_q < i0 + kRows ? a->n_q : i0 + kRows;
      int64_t s0 = k_lo + span * s / splits, s1 = k_lo + span * (s + 1) / splits;
      int64_t lo0 = lo_of(a, a->pos0 + i0);
      int64_t r0 = s0 > lo0 ? s0 : lo0;
      int64_t r1 = s1 < a->pos0 + i1 ? s1 : a->pos0 + i1;
      for (int i = 0; i < kRows; ++i)
        for (int g = 0; g < kMaxGroup; ++g) {
          st_m[i][g] = neg_inf;
          st_l[i][g] = 0.f;
        }
      memset(acc, 0, sizeof(float) * acc_per_task);
      for (int64_t kp = r0; kp < r1; kp += kTile) {
        int64_t kq = r1 < kp + kTile ? r1 : kp + kTile;
        int64_t cut = a->pos0 > kp ? a->pos0 : kp;
        if (cut > kq) cut = kq;
        if (cut > kp) xo_kv_load(a->cache, h, kp, cut, kt, vt);
        for (int64_t p = cut; p < kq; ++p) {
          const size_t src = ((size_t)(p - a->pos0) * (size_t)a->kv_heads + (size_t)h) * (size_t)d;
          memcpy(kt + (size_t)(p - kp) * (size_t)d, a->k + src, sizeof(float) * (size_t)d);
          memcpy(vt + (size_t)(p - kp) * (size_t)d, a->v + src, sizeof(float) * (size_t)d);
        }
        for (int i = i0; i < i1; ++i) {
          int64_t t = a->pos0 + i;
          int64_t lt = lo_of(a, t);
          int64_t j0 = kp > lt ? kp : lt, j1 = kq < t + 1 ? kq : t + 1;
          if (j0 >= j1) continue;
          for (int g = 0; g < group; ++g) {
            const float* qv = a->q + ((size_t)i * (size_t)a->heads + (size_t)(h * group + g)) * (size_t)d;
            float mx = neg_inf;
            for (int64_t j = j0; j < j1; ++j) {
              const float* kv = kt + (size_t)(j - kp) * (size_t)d;
              float dot = dot_f32(qv, kv, d) * a->scale;
              sc[j - j0] = dot;
              mx = fmaxf(mx, dot);
            }
            float* m = &st_m[i - i0][g];
            float* l = &st_l[i - i0][g];
            float m_new = fmaxf(*m, mx);
            float corr = *m == neg_inf ? 0.f : expf(*m - m_new);
            float* ac = acc + ((size_t)(i - i0) * (size_t)group + (size_t)g) * (size_t)d;
            if (corr != 1.f)
              for (int e = 0; e < d; ++e) ac[e] *= corr;
            *l *= corr;
            for (int64_t j = j0; j < j1; ++j) {
              float w = expf(sc[j - j0] - m_new);
              *l += w;
              const float* vv = vt + (size_t)(j - kp) * (size_t)d;
              for (int e = 0; e < d; ++e) ac[e] += w * vv[e];
            }
            *m = m_new;
          }
        }
      }
      if (splits == 1) {
        for (int i = i0; i < i1; ++i)
          for (int g = 0; g < group; ++g) {
            float* o = a->out + ((size_t)i * (size_t)a->heads + (size_t)(h * group + g)) * (size_t)d;
            const float* ac = acc + ((size_t)(i - i0) * (size_t)group + (size_t)g) * (size_t)d;
            float l = st_l[i - i0][g];
            float inv = l > 0.f ? 1.f / l : 0.f;
            for (int e = 0; e < d; ++e) o[e] = ac[e] * inv;
          }
      } else {
        memcpy(part_m + (size_t)task * kRows * kMaxGroup, st_m, sizeof(st_m));
        memcpy(part_l + (size_t)task * kRows * kMaxGroup, st_l, sizeof(st_l));
        memcpy(accs + (size_t)task * acc_per_task, acc, sizeof(float) * acc_per_task);
      }
    }
    free(kt);
    free(vt);
    free(acc);
  }
  if (splits > 1) {
    /* engine/src/kv.cpp:262-285 */
    for (int h = 0; h < a->kv_heads; ++h)
      for (int qb = 0; qb < qblocks; ++qb) {
        int i0 = qb * kRows, i1 = a->n_q < i0 + kRows ? a->n_q : i0 + kRows;
        int64_t base = ((int64_t)h * qblocks + qb) * splits;
        for (int i = i0; i < i1; ++i)
          for (int g = 0; g < group; ++g) {
            float mx = neg_inf;
            for (int s = 0; s < splits; ++s)
              mx = fmaxf(mx, part_m[(size_t)(base + s) * kRows * kMaxGroup + (size_t)(i - i0) * kMaxGroup + g]);
            float* o = a->out + ((size_t)i * (size_t)a->heads + (size_t)(h * group + g)) * (size_t)d;
            for (int e = 0; e < d; ++e) o[e] = 0.f;
            float l = 0.f;
            for (int s = 0; s < splits; ++s) {
              size_t pi = (size_t)(base + s) * kRows * kMaxGroup + (size_t)(i - i0) * kMaxGroup + g;
              if (part_l[pi] == 0.f) continue;
              float w = expf(part_m[pi] - mx);
              l += w * part_l[pi];
              const float* ac = accs + (size_t)(base + s) * acc_per_task +
                                ((size_t)(i - i0) * (size_t)group + (size_t)g) * (size_t)d;
              for (int e = 0; e < d; ++e) o[e] += w * ac[e];
            }
            float inv = l > 0.f ? 1.f / l : 0.f;
            for (int e = 0; e < d; ++e) o[e] *= inv;
          }
      }
  }
  free(part_m);
  free(part_l);
  free(accs);
  return 0;
}

int xo_attention_slots(const xo_attn_args* a, const int64_t* slot_pos, int threads) {
  /* npu/xtg_npu.cpp:236-258 mask semantics (slot visibility from the stored positions), evaluated with the
   * CPU kernel's arithmetic (FP32 dot_f32 scores, online softmax over tiles of 64 keys, kv.cpp:205-245):
   * the ring's slots in slot order, then this call's own keys in order. */
  const int group = a->heads / a->kv_heads, d = a->head_dim;
  if (group * a->kv_heads != a->heads || group > kMaxGroup) return -1;
  if (threads < 1) threads = 1;
  const int64_t slots = a->cache->slots;
  const int64_t total = slots + a->n_q;
  const int64_t tasks = (int64_t)a->n_q * a->heads;
#pragma omp parallel num_threads(threads)
  {
    float* kt = (float*)malloc(sizeof(float) * (size_t)d);
    float* vt = (float*)malloc(sizeof(float) * (size_t)d);
    float* acc = (float*)malloc(sizeof(float) * (size_t)d);
    float* kk = (float*)malloc(sizeof(float) * (size_t)kTile * (size_t)d);
    float* vv = (float*)malloc(sizeof(float) * (size_t)kTile * (size_t)d);
    float sc[kTile];
    int ok[kTile];
#pragma omp for schedule(dynamic, 1)
    for (int64_t task = 0; task < tasks; ++task) {
      int i = (int)(task / a->heads), hq = (int)(task % a->heads), h = hq / group;
      int64_t p = a->pos0 + i;
      const float* qv = a->q + ((size_t)i * (size_t)a->heads + (size_t)hq) * (size_t)d;
      float m = -INFINITY, l = 0.f;
      memset(acc, 0, sizeof(float) * (size_t)d);
      for (int64_t t0 = 0; t0 < total; t0 += kTile) {
        int64_t t1 = total < t0 + kTile ? total : t0 + kTile;
        float mx = -INFINITY;
        for (int64_t t = t0; t < t1; ++t) {
          int see;
          if (t < slots) {
            int64_t q = slot_pos[t];
            see = q >= 0 && q < a->pos0 && (a->window <= 0 || p - q < a->window);
            if (see) {
              xo_kv_load(a->cache, h, q, q + 1, kt, vt);
              memcpy(kk + (size_t)(t - t0) * (size_t)d, kt, sizeof(float) * (size_t)d);
              memcpy(vv + (size_t)(t - t0) * (size_t)d, vt, sizeof(float) * (size_t)d);
            }
          } else {
            int j = (int)(t - slots);
            see = j <= i && (a->window <= 0 || i - j < a->window);
            if (see) {
              const size_t src = ((size_t)j * (size_t)a->kv_heads + (size_t)h) * (size_t)d;
              memcpy(kk + (size_t)(t - t0) * (size_t)d, a->k + src, sizeof(float) * (size_t)d);
              memcpy(vv + (size_t)(t - t0) * (size_t)d, a->v + src, sizeof(float) * (size_t)d);
            }
          }
          ok[t - t0] = see;
          if (see) {
            float dot = dot_f32(qv, kk + (size_t)(t - t0) * (size_t)d, d) * a->scale;
            sc[t - t0] = dot;
            mx = fmaxf(mx, dot);
          }
        }
        if (mx == -INFINITY) continue;
        float m_new = fmaxf(m, mx);
        float corr = m == -INFINITY ? 0.f : expf(m - m_new);
        if (corr != 1.f)
          for (int e = 0; e < d; ++e) acc[e] *= corr;
        l *= corr;
        for (int64_t t = t0; t < t1; ++t) {
          if (!ok[t - t0]) continue;
          float w = expf(sc[t - t0] - m_new);
          l += w;
          const float* vr = vv + (size_t)(t - t0) * (size_t)d;
          for (int e = 0; e < d; ++e) acc[e] += w * vr[e];
        }
        m = m_new;
      }
      float* o = a->out + ((size_t)i * (size_t)a->heads + (size_t)hq) * (size_t)d;
      float inv = l > 0.f ? 1.f / l : 0.f;
      for (int e = 0; e < d; ++e) o[e] = acc[e] * inv;
    }
    free(kt);
    free(vt);
    free(acc);
    free(kk);
    free(vv);
  }
  return 0;
}

/* -------------------------------------------------------------------------------------------- decode step */

struct xo_dory {
  xo_dory_config c;
  const xo_dory_layer* layers;
  const xo_nvfp4* head;
  const uint16_t* head_bf16; /* [vocab][hidden] BF16, or NULL */
  const float* logit_scale;
  int n_layers, n_attn;
  int* attn_of;    /* per sublayer: its attention index, or -1 */
  xo_kv** caches;  /* [n_attn][loops] (instance 0 only for non-recurrent sublayers) */
};

static int xo_recurrent(const xo_dory* d, int l) { return l >= d->c.n_in && l < d->c.n_in + d->c.n_rec; }

xo_dory* xo_dory_create(const xo_dory_config* c, const xo_dory_layer* layers, const xo_nvfp4* head,
                        const float* logit_scale) {
  /* the session's caches: packs/dory/dory.cpp:436-447 (per_loop: one cache per loop for recurrent sublayers;
   * last_loop: one) */
  xo_dory* d = (xo_dory*)calloc(1, sizeof(xo_dory));
  d->c = *c;
  d->layers = layers;
  d->head = head;
  d->logit_scale = logit_scale;
  d->n_layers = c->n_in + c->n_rec + c->n_out;
  d->attn_of = (int*)malloc(sizeof(int) * (size_t)d->n_layers);
  for (int l = 0; l < d->n_layers; ++l) d->attn_of[l] = layers[l].kind == XO_MLP ? -1 : d->n_attn++;
  d->caches = (xo_kv**)calloc((size_t)d->n_attn * (size_t)c->loops, sizeof(xo_kv*));
  for (int l = 0; l < d->n_layers; ++l) {
    if (d->attn_of[l] < 0) continue;
    int inst = xo_recurrent(d, l) && c->kv_mode != XO_KV_LAST_LOOP ? c->loops : 1;
    for (int i = 0; i < inst; ++i)
      d->caches[(size_t)d->attn_of[l] * (size_t)c->loops + (size_t)i] =
          xo_kv_create(c->kv_heads, c->head_dim, c->context, layers[l].kind == XO_SLIDING ? c->ring_slots : 0,
                       c->kv_dtype);
  }
  return d;
}

void xo_dory_free(xo_dory* d) {
  if (!d) return;
  for (int i = 0; i < d->n_attn * d->c.loops; ++i) xo_kv_free(d->caches[i]);
  free(d->caches);
  free(d->attn_of);
  free(d);
}

void xo_dory_head_bf16(xo_dory* d, const uint16_t* w) { d->head_bf16 = w; }

xo_kv* xo_dory_cache(xo_dory* d, int attn, int inst) {
  if (attn < 0 || attn >= d->n_attn || inst < 0 || inst >= d->c.loops) return NULL;
  return d->caches[(size_t)attn * (size_t)d->c.loops + (size_t)inst];
}

typedef struct {
  float *mg, *mu, *hq, *hk, *hv, *hg, *ha, *ho;
} xo_scratch;

static void xo_sublayer(xo_dory* d, int l, float* x, int m, int64_t pos0, int inst, int store, xo_scratch* s,
                        int threads) {
  /* packs/dory/dory.cpp:467-518 */
  const xo_dory_config* c = &d->c;
  const xo_dory_layer* L = &d->layers[l];
  const int H = c->hidden, Q = c->heads * c->head_dim;
  if (L->kind == XO_MLP) {
    xo_nvfp4 gu[2] = {L->gate, L->up};
    float* ys[2] = {s->mg, s->mu};
    xo_matmul_nvfp4(gu, 2, x, m, ys, threads);
    xo_swiglu_scaled(s->mg, s->mu, L->sg, L->su, m, c->ffn);
    xo_justnorm(s->mg, m, c->ffn);
    float* yo[1] = {s->ho};
    xo_matmul_nvfp4(&L->down, 1, s->mg, m, yo, threads);
    xo_slerp_residual(x, s->ho, L->lr, m, H);
    return;
  }
  xo_nvfp4 qkvg[4] = {L->q, L->k, L->v, L->g};
  float* ys[4] = {s->hq, s->hk, s->hv, s->hg};
  xo_matmul_nvfp4(qkvg, 4, x, m, ys, threads);
  const float theta = L->kind == XO_SLIDING ? c->theta_sliding : c->theta_full;
  xo_qk_produce(s->hq, s->hk, m, c->heads, c->kv_heads, c->head_dim, pos0, theta, L->qscale);
  xo_kv* cache = xo_dory_cache(d, d->attn_of[l], inst);
  xo_attn_args a;
  a.n_q = m;
  a.pos0 = pos0;
  a.heads = c->heads;
  a.kv_heads = c->kv_heads;
  a.head_dim = c->head_dim;
  a.window = L->kind == XO_SLIDING ? c->window : 0;
  a.scale = 1.f / sqrtf((float)c->head_dim);
  a.q = s->hq;
  a.k = s->hk;
  a.v = s->hv;
  a.cache = cache;
  a.out = s->ha;
  xo_attention(&a, threads, threads);
  if (store) xo_kv_store(cache, pos0, m, s->hk, s->hv);
  xo_gate_norm(s->ha, s->hg, L->gscale, m, Q);
  float* yo[1] = {s->ho};
  xo_matmul_nvfp4(&L->o, 1, s->ha, m, yo, threads);
  xo_slerp_residual(x, s->ho, L->lr, m, H);
}

int xo_dory_forward(xo_dory* d, const float* x, int m, int64_t pos0, float* logits, int threads) {
  /* packs/dory/dory.cpp:520-544 (run_chunk after the embedding rows) and :566-576 (head, logit scale) */
  const xo_dory_config* c = &d->c;
  const int H = c->hidden, Q = c->heads * c->head_dim, KV = c->kv_heads * c->head_dim;
  const size_t n = (size_t)m * (size_t)H;
  xo_scratch s;
  s.mg = (float*)malloc(sizeof(float) * (size_t)m * (size_t)c->ffn);
  s.mu = (float*)malloc(sizeof(float) * (size_t)m * (size_t)c->ffn);
  s.hq = (float*)malloc(sizeof(float) * (size_t)m * (size_t)Q);
  s.hk = (float*)malloc(sizeof(float) * (size_t)m * (size_t)KV);
  s.hv = (float*)malloc(sizeof(float) * (size_t)m * (size_t)KV);
  s.hg = (float*)malloc(sizeof(float) * (size_t)m * (size_t)Q);
  s.ha = (float*)malloc(sizeof(float) * (size_t)m * (size_t)Q);
  s.ho = (float*)malloc(sizeof(float) * n);
  float* xs = (float*)malloc(sizeof(float) * n);
  float* input = (float*)malloc(sizeof(float) * n);
  float* state = (float*)malloc(sizeof(float) * n);
  memcpy(xs, x, sizeof(float) * n);
  int l = 0;
  for (; l < c->n_in; ++l) xo_sublayer(d, l, xs, m, pos0, 0, 1, &s, threads);
  memcpy(input, xs, sizeof(float) * n);
  memcpy(state, xs, sizeof(float) * n);
  for (int i = 0; i < c->loops; ++i) {
    for (size_t j = 0; j < n; ++j) xs[j] = state[j] + input[j];
    xo_justnorm(xs, m, H);
    /* last_loop: every loop attends to this chunk's own keys, the cache keeps the last loop's (dory.cpp:534-537) */
    const int last_loop = c->kv_mode == XO_KV_LAST_LOOP;
    const int store = !last_loop || i == c->loops - 1;
    for (int r = c->n_in; r < c->n_in + c->n_rec; ++r)
      xo_sublayer(d, r, xs, m, pos0, last_loop ? 0 : i, store, &s, threads);
    memcpy(state, xs, sizeof(float) * n);
    xo_justnorm(state, m, H);
  }
  memcpy(xs, state, sizeof(float) * n);
  for (l = c->n_in + c->n_rec; l < d->n_layers; ++l) xo_sublayer(d, l, xs, m, pos0, 0, 1, &s, threads);
  if (d->head_bf16) { /* the BF16 checkpoint's head (dory.cpp:325, 401-402: matmul_bf16) */
    xo_matmul_bf16(d->head_bf16, c->vocab, H, xs, m, logits, threads);
  } else {
    float* yl[1] = {logits};
    xo_matmul_nvfp4(d->head, 1, xs, m, yl, threads);
  }
  for (int r = 0; r < m; ++r) {
    float* lg = logits + (size_t)r * (size_t)c->vocab;
    for (int j = 0; j < c->vocab; ++j) lg[j] *= d->logit_scale[j];
  }
  free(s.mg);
  free(s.mu);
  free(s.hq);
  free(s.hk);
  free(s.hv);
  free(s.hg);
  free(s.ha);
  free(s.ho);
  free(xs);
  free(input);
  free(state);
  return 0;
}
