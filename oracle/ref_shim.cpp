// extern "C" entry points into the reference engine's own CPU kernels, compiled from the reference sources by
// oracle/Makefile into oracle/_ref/libxtgref.so. TEST INFRASTRUCTURE ONLY: used to pin the oracle restatement
// and, when present, as the CPU baseline. Calls go straight to xtg::matmul_nvfp4 / attention / KvCache / rope /
// justnorm / slerp_residual / swiglu_scaled / f32_to_e4m3 / argmax (engine/include/xtg/{fp,kernels,kv,sampler}.h),
// and to the Dory pack's own CPU session (packs/dory/dory.cpp: load_model -> DoryModel -> DorySession::forward).
#include <cstdint>
#include <cstring>
#include <limits>
#include <map>
#include <random>
#include <memory>
#include <string>
#include <vector>

#include "xtg/common.h"
#include "xtg/fp.h"
#include "xtg/kernels.h"
#include "xtg/kv.h"
#include "xtg/model.h"
#include "xtg/sampler.h"
#include "xtg/threadpool.h"

namespace xtg {
void register_builtin_packs();   // packs/packs.cpp
}

namespace {
xtg::ThreadPool& pool_of(int threads) {
  static std::map<int, std::unique_ptr<xtg::ThreadPool>> pools;
  auto& p = pools[threads];
  if (!p) p = std::make_unique<xtg::ThreadPool>(threads);
  return *p;
}
}  // namespace

extern "C" {

// Same field order as xtg::Nvfp4Weight.
struct xr_nvfp4 {
  const uint8_t* codes;
  const uint8_t* scales;
  float global;
  int n_out, k;
};

float xr_e4m3_to_f32(uint8_t b) { return xtg::e4m3_to_f32(b); }
uint8_t xr_f32_to_e4m3(float f) { return xtg::f32_to_e4m3(f); }
uint16_t xr_f32_to_bf16(float f) { return xtg::f32_to_bf16(f); }
float xr_bf16_to_f32(uint16_t h) { return xtg::bf16_to_f32(h); }

void xr_nvfp4_row(const xr_nvfp4* w, int n, float* out) {
  xtg::Nvfp4Weight r{w->codes, w->scales, w->global, w->n_out, w->k};
  xtg::nvfp4_row(r, n, out);
}

int xr_matmul_nvfp4(const xr_nvfp4* ws, int n_w, const float* x, int m, float* const* ys, int threads) {
  try {
    std::vector<xtg::Nvfp4Weight> w(static_cast<size_t>(n_w));
    std::vector<const xtg::Nvfp4Weight*> wp;
    std::vector<float*> yp;
    for (int i = 0; i < n_w; ++i) {
      w[size_t(i)] = {ws[i].codes, ws[i].scales, ws[i].global, ws[i].n_out, ws[i].k};
      wp.push_back(&w[size_t(i)]);
      yp.push_back(ys[i]);
    }
    xtg::matmul_nvfp4(pool_of(threads), wp, x, m, yp);
    return 0;
  } catch (...) {
    return -1;
  }
}

int xr_matmul_bf16(const uint16_t* w, int n_out, int k, const float* x, int m, float* y, int threads) {
  try {
    xtg::Bf16Weight b{w, n_out, k};
    xtg::matmul_bf16(pool_of(threads), b, x, m, y);
    return 0;
  } catch (...) {
    return -1;
  }
}

void xr_justnorm(float* x, int rows, int width) { xtg::justnorm(x, rows, width); }
int xr_argmax(const float* x, int n) { return xtg::argmax(x, n); }
// The reference Sampler seeded with `seed` samples one row; *u gets the draw its uniform_real_distribution made
// (generate_canonical<double, 53> of a generator seeded alike), which a caller hands to a sampler that takes u.
int xr_sample(const float* x, int n, float temperature, float top_p, int top_k, float min_p, uint64_t seed,
              double* u) {
  xtg::SamplingParams p;
  p.temperature = temperature;
  p.top_p = top_p;
  p.top_k = top_k;
  p.min_p = min_p;
  xtg::Sampler s(seed);
  std::mt19937_64 g(seed);
  *u = std::generate_canonical<double, std::numeric_limits<double>::digits>(g);
  return s.sample(x, n, p);
}
void xr_slerp_residual(float* a, const float* b, const float* lr, int rows, int width) {
  xtg::slerp_residual(a, b, lr, rows, width);
}
void xr_rope(float* x, int rows, int heads, int head_dim, int64_t pos0, float theta) {
  xtg::rope(x, rows, heads, head_dim, pos0, theta);
}
void xr_swiglu_scaled(float* g, const float* u, const float* sg, const float* su, int rows, int w) {
  xtg::swiglu_scaled(g, u, sg, su, rows, w);
}

void* xr_kv_create(int kv_heads, int head_dim, int64_t slots, int ring, int fp8) {
  try {
    return new xtg::KvCache(kv_heads, head_dim, slots, ring, fp8 ? xtg::KvDtype::FP8 : xtg::KvDtype::BF16);
  } catch (...) {
    return nullptr;
  }
}
void xr_kv_free(void* c) { delete static_cast<xtg::KvCache*>(c); }
int xr_kv_store(void* c, int64_t pos, int n, const float* k, const float* v) {
  try {
    static_cast<xtg::KvCache*>(c)->store(pos, n, k, v);
    return 0;
  } catch (...) {
    return -1;
  }
}
void xr_kv_load(const void* c, int h, int64_t p0, int64_t p1, float* k, float* v) {
  static_cast<const xtg::KvCache*>(c)->load(h, p0, p1, k, v);
}

struct xr_attn_args {
  int n_q;
  int64_t pos0;
  int heads, kv_heads, head_dim;
  int window;
  float scale;
  const float* q;
  const float* k;
  const float* v;
  const void* cache;
  float* out;
};

int xr_attention(const xr_attn_args* a, int threads) {
  try {
    xtg::AttnArgs r;
    r.n_q = a->n_q;
    r.pos0 = a->pos0;
    r.heads = a->heads;
    r.kv_heads = a->kv_heads;
    r.head_dim = a->head_dim;
    r.window = a->window;
    r.scale = a->scale;
    r.q = a->q;
    r.k = a->k;
    r.v = a->v;
    r.cache = static_cast<const xtg::KvCache*>(a->cache);
    r.out = a->out;
    xtg::attention(pool_of(threads), r);
    return 0;
  } catch (...) {
    return -1;
  }
}

// --- the Dory pack's CPU session (packs/dory/dory.cpp:304-578), as the server drives it (model.h:31-63) ---

struct xr_dory {
  std::unique_ptr<xtg::Model> model;
  std::unique_ptr<xtg::Session> session;
};

static void put_err(const char* what, char* err, int err_len) {
  if (err && err_len > 0) {
    std::strncpy(err, what, size_t(err_len) - 1);
    err[err_len - 1] = 0;
  }
}

// load_model(dir, options) (engine/src/model.cpp:35-38) on a checkpoint directory, then one session. options is
// the pack's launch-option JSON (dory.cpp:136-170), e.g. {"backend": "cpu", "kv_dtype": "bf16", "loops": 2}.
void* xr_dory_open(const char* dir, const char* options, int threads, int* vocab, char* err, int err_len) {
  try {
    xtg::register_builtin_packs();
    auto d = std::make_unique<xr_dory>();
    d->model = xtg::load_model(dir, xtg::json::parse(options && *options ? options : "{}"), pool_of(threads));
    d->session = d->model->new_session();
    *vocab = d->model->info().vocab;
    return d.release();
  } catch (const std::exception& e) {
    put_err(e.what(), err, err_len);
    return nullptr;
  }
}

void xr_dory_close(void* h) { delete static_cast<xr_dory*>(h); }

// Session::forward(tokens, n, want, on_logits): the n tokens at positions n_past() .. ; logits receives the rows
// on_logits hands over, in order (want 0 none, 1 the last row, 2 every row: xtg::Logits). Returns the rows written.
int xr_dory_forward(void* h, const int32_t* tokens, int n, int want, float* logits, char* err, int err_len) {
  try {
    auto* d = static_cast<xr_dory*>(h);
    const int vocab = d->model->info().vocab;
    int rows = 0;
    const xtg::Logits w = want == 2 ? xtg::Logits::All : want == 1 ? xtg::Logits::Last : xtg::Logits::None;
    d->session->forward(tokens, n, w, [&](int, const float* lg) {
      std::memcpy(logits + size_t(rows) * size_t(vocab), lg, size_t(vocab) * sizeof(float));
      rows += 1;
    });
    return rows;
  } catch (const std::exception& e) {
    put_err(e.what(), err, err_len);
    return -1;
  }
}

int64_t xr_dory_n_past(void* h) { return static_cast<xr_dory*>(h)->session->n_past(); }
int xr_dory_rewind(void* h, int64_t n) { return static_cast<xr_dory*>(h)->session->rewind(n) ? 1 : 0; }
void xr_dory_snapshot(void* h, int slot) { static_cast<xr_dory*>(h)->session->snapshot(slot); }
int xr_dory_restore(void* h, int slot) { return static_cast<xr_dory*>(h)->session->restore(slot) ? 1 : 0; }

}  // extern "C"
