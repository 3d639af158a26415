// The C ABI of include/xtg_hip.h: every entry point catches what the backend throws and returns -1 (or NULL)
// with the message in err, as the reference's plugin ABI does (npu/xtg_npu.cpp:517-526, server/capi.cpp:23-35).
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <string>

#include "backend.hpp"
#include "common.hpp"
#include "dory.hpp"
#include "xtg_hip.h"

struct xtg_hip {
  std::unique_ptr<xtg::hip::Backend> b;
};

static_assert(XTG_HIP_ATTN_SCRATCH_BYTES == xtg::hip::kAttnScratchBytes, "the header's scratch size is the kernel's");

namespace {
void put_err(char* err, int err_len, const char* msg) {
  if (err && err_len > 0) {
    std::snprintf(err, size_t(err_len), "%s", msg);
  }
}

template <class F>
int guarded(char* err, int err_len, F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    put_err(err, err_len, e.what());
  } catch (...) {
    put_err(err, err_len, "unknown error");
  }
  return -1;
}

int option_int(const char* json, const char* key, int def) {
  if (!json) return def;
  std::string s(json), k = std::string("\"") + key + "\"";
  size_t p = s.find(k);
  if (p == std::string::npos) return def;
  p = s.find(':', p + k.size());
  if (p == std::string::npos) return def;
  return std::atoi(s.c_str() + p + 1);
}
}  // namespace

extern "C" {

xtg_hip* xtg_hip_open(const char* options, char* err, int err_len) {
  xtg_hip* h = nullptr;
  int rc = guarded(err, err_len, [&] {
    auto b = std::make_unique<xtg::hip::Backend>(option_int(options, "device", 0));
    h = new xtg_hip{std::move(b)};
  });
  return rc == 0 ? h : nullptr;
}

void xtg_hip_close(xtg_hip* h) {
  try {
    delete h;
  } catch (...) {
  }
}

int xtg_hip_info(xtg_hip* h, char* out, int out_len) {
  if (!h) return -1;
  std::string s;
  if (guarded(nullptr, 0, [&] { s = h->b->info_json(); }) != 0) return -1;
  if (out && out_len > 0) std::snprintf(out, size_t(out_len), "%s", s.c_str());
  return int(s.size());
}

void* xtg_hip_stream(xtg_hip* h) { return h ? static_cast<void*>(h->b->stream()) : nullptr; }

int xtg_hip_prepare_nvfp4(xtg_hip* h, const xtg_nvfp4* w, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && w, "prepare: NULL handle or weight");
    h->b->prepare(*w);
  });
}

int xtg_hip_release_nvfp4(xtg_hip* h, const uint8_t* codes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "release_nvfp4: NULL handle");
    h->b->release_weight(codes);
  });
}

int xtg_hip_matmul_nvfp4(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const float* x, int m, float* const* ys, char* err,
                         int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && ws && ys, "matmul: NULL argument");
    h->b->matmul(ws, n_w, x, m, ys);
  });
}

int xtg_hip_matmul_nvfp4_dev(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const void* x, int x_dtype, int m, float* y,
                             size_t y_offset, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && ws, "matmul: NULL argument");
    h->b->matmul_dev(ws, n_w, x, x_dtype, m, y, y_offset);
  });
}

int xtg_hip_prepare_bf16(xtg_hip* h, const xtg_bf16* w, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && w, "prepare_bf16: NULL argument");
    h->b->prepare(*w);
  });
}

int xtg_hip_release_bf16(xtg_hip* h, const uint16_t* data, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "release_bf16: NULL handle");
    h->b->release_bf16(data);
  });
}

int xtg_hip_matmul_bf16(xtg_hip* h, const xtg_bf16* w, const float* x, int m, float* y, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && w && x && y, "matmul_bf16: NULL argument");
    h->b->matmul_bf16(*w, x, m, y);
  });
}

int xtg_hip_matmul_bf16_dev(xtg_hip* h, const xtg_bf16* w, const void* x, int x_dtype, int m, float* y,
                            size_t y_offset, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && w, "matmul_bf16: NULL argument");
    h->b->matmul_bf16_dev(*w, x, x_dtype, m, y, y_offset);
  });
}

xtg_hip_kv* xtg_hip_kv_create(xtg_hip* h, int kv_heads, int head_dim, int64_t slots, int ring, int dtype, char* err,
                              int err_len) {
  xtg::hip::DevKv* c = nullptr;
  int rc = guarded(err, err_len, [&] {
    XTG_CHECK(h, "kv_create: NULL handle");
    c = h->b->kv_create(kv_heads, head_dim, slots, ring, dtype);
  });
  return rc == 0 ? reinterpret_cast<xtg_hip_kv*>(c) : nullptr;
}

void xtg_hip_kv_destroy(xtg_hip* h, xtg_hip_kv* kv) {
  if (h && kv) guarded(nullptr, 0, [&] { h->b->kv_destroy(reinterpret_cast<xtg::hip::DevKv*>(kv)); });
}

int xtg_hip_kv_store(xtg_hip* h, xtg_hip_kv* kv, int64_t pos, int n, const float* k, const float* v, char* err,
                     int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && kv, "kv_store: NULL argument");
    h->b->kv_store(reinterpret_cast<xtg::hip::DevKv*>(kv), pos, n, k, v);
  });
}

int xtg_hip_kv_load(xtg_hip* h, const xtg_hip_kv* kv, int head, int64_t p0, int64_t p1, float* k, float* v, char* err,
                    int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && kv && k && v, "kv_load: NULL argument");
    h->b->kv_load(reinterpret_cast<const xtg::hip::DevKv*>(kv), head, p0, p1, k, v);
  });
}

int64_t xtg_hip_kv_bytes(xtg_hip* h, const xtg_hip_kv* kv) {
  if (!h || !kv) return -1;
  return int64_t(h->b->kv_bytes(reinterpret_cast<const xtg::hip::DevKv*>(kv)));
}

int xtg_hip_kv_save(xtg_hip* h, const xtg_hip_kv* kv, void* out, size_t bytes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && kv && out, "kv_save: NULL argument");
    h->b->kv_save(reinterpret_cast<const xtg::hip::DevKv*>(kv), out, bytes);
  });
}

int xtg_hip_kv_restore(xtg_hip* h, xtg_hip_kv* kv, const void* in, size_t bytes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && kv && in, "kv_restore: NULL argument");
    h->b->kv_restore(reinterpret_cast<xtg::hip::DevKv*>(kv), in, bytes);
  });
}

int xtg_hip_kv_release(xtg_hip* h, xtg_hip_kv* kv, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && kv, "kv_release: NULL argument");
    h->b->kv_release(reinterpret_cast<xtg::hip::DevKv*>(kv));
  });
}

int xtg_hip_nvfp4_tiles(xtg_hip* h, const uint8_t* codes, void* out, size_t bytes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && codes && out, "nvfp4_tiles: NULL argument");
    h->b->read_tiles(codes, out, bytes);
  });
}

int xtg_hip_kv_copy(xtg_hip* h, const xtg_hip_kv* src, xtg_hip_kv* dst, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && src && dst, "kv_copy: NULL argument");
    h->b->kv_copy(reinterpret_cast<const xtg::hip::DevKv*>(src), reinterpret_cast<xtg::hip::DevKv*>(dst));
  });
}

int xtg_hip_attention(xtg_hip* h, const xtg_attn_args* a, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && a && a->cache, "attention: NULL argument");
    const auto* c = reinterpret_cast<const xtg::hip::DevKv*>(a->cache);
    XTG_CHECK(a->kv_heads == c->kv_heads && a->head_dim == c->head_dim,
              "attention: %d KV heads of %d for a cache of %d of %d", a->kv_heads, a->head_dim, c->kv_heads,
              c->head_dim);
    h->b->attention(c, a->n_q, a->pos0, a->heads, a->window, a->scale, a->q, a->k, a->v, a->out);
  });
}

int xtg_hip_attention_noalloc(xtg_hip* h, const xtg_attn_args* a, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && a && a->cache, "attention_noalloc: NULL argument");
    const auto* c = reinterpret_cast<const xtg::hip::DevKv*>(a->cache);
    XTG_CHECK(a->kv_heads == c->kv_heads && a->head_dim == c->head_dim,
              "attention_noalloc: %d KV heads of %d for a cache of %d of %d", a->kv_heads, a->head_dim, c->kv_heads,
              c->head_dim);
    h->b->attention_noalloc(c, a->n_q, a->pos0, a->heads, a->window, a->scale, a->q, a->k, a->v, a->out);
  });
}

int xtg_hip_qk_rope_norm(xtg_hip* h, float* q, float* k, int m, int heads, int kv_heads, int head_dim, int64_t pos0,
                         float theta, const float* qscale, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "rope: NULL handle");
    h->b->qk_rope_norm(q, k, m, heads, kv_heads, head_dim, pos0, theta, qscale);
  });
}

int xtg_hip_slerp_residual(xtg_hip* h, float* x, const float* o, const float* lr, int rows, int width, char* err,
                           int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "slerp: NULL handle");
    h->b->slerp_norm(x, o, lr, rows, width);
  });
}

int xtg_hip_swiglu_norm(xtg_hip* h, float* g, const float* u, const float* sg, const float* su, int rows, int width,
                        char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "swiglu: NULL handle");
    h->b->swiglu_norm(g, u, sg, su, rows, width, g);
  });
}

int xtg_hip_gate_norm(xtg_hip* h, float* att, const float* gate, const float* gs, int rows, int width, char* err,
                      int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "gate_norm: NULL handle");
    h->b->gate_norm(att, gate, gs, rows, width, att);
  });
}

int xtg_hip_add_norm(xtg_hip* h, const float* a, const float* b, float* out, int rows, int width, char* err,
                     int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "add_norm: NULL handle");
    h->b->add_norm(a, b, out, rows, width);
  });
}

int xtg_hip_argmax(xtg_hip* h, const float* logits, int rows, int n, int32_t* out, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "argmax: NULL handle");
    h->b->argmax(logits, rows, n, out);
  });
}

int xtg_hip_sample(xtg_hip* h, const float* logits, int rows, int n, const xtg_sampling* p, const double* u,
                   int32_t* out, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && p, "sample: NULL handle or parameters");
    h->b->sample(logits, rows, n, p->temperature, p->top_p, p->top_k, p->min_p, u, out);
  });
}

struct xtg_hip_dory {
  xtg_hip* h;
  std::unique_ptr<xtg::hip::DorySession> s;
};

xtg_hip_dory* xtg_hip_dory_create(xtg_hip* h, const xtg_dory_config* c, const xtg_dory_layer* layers,
                                  const xtg_nvfp4* head, const float* logit_scale, char* err, int err_len) {
  xtg_hip_dory* d = nullptr;
  int rc = guarded(err, err_len, [&] {
    XTG_CHECK(h && c && layers && logit_scale, "dory_create: NULL argument");
    const xtg_nvfp4 none{nullptr, nullptr, 1.f, 0, 0};
    auto s = std::make_unique<xtg::hip::DorySession>(*h->b, *c, layers, head ? *head : none, logit_scale);
    d = new xtg_hip_dory{h, std::move(s)};
  });
  return rc == 0 ? d : nullptr;
}

int xtg_hip_dory_head_bf16(xtg_hip_dory* d, const xtg_bf16* head, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(d && head, "dory_head_bf16: NULL argument");
    XTG_CHECK(!d->h->b->capturing(), "dory_head_bf16: not during a graph capture");
    d->s->set_head_bf16(*head);
  });
}

void xtg_hip_dory_destroy(xtg_hip_dory* d) {
  try {
    delete d;
  } catch (...) {
  }
}

int xtg_hip_dory_forward(xtg_hip_dory* d, const float* x, int m, int64_t pos0, float* logits, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(d && x && logits, "dory_forward: NULL argument");
    d->s->forward(x, m, pos0, logits);
  });
}

int xtg_hip_dory_prefill(xtg_hip_dory* d, const float* x, int n, int64_t pos0, int want, float* logits, char* err,
                         int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(d && x, "dory_prefill: NULL argument");
    d->s->prefill(x, n, pos0, want, logits);
  });
}

int xtg_hip_dory_snapshot(xtg_hip_dory* d, int slot, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(d, "dory_snapshot: NULL handle");
    d->s->snapshot(slot);
  });
}

int xtg_hip_dory_restore(xtg_hip_dory* d, int slot, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(d, "dory_restore: NULL handle");
    d->s->restore(slot);
  });
}

xtg_hip_kv* xtg_hip_dory_cache(xtg_hip_dory* d, int attn, int inst) {
  xtg::hip::DevKv* c = nullptr;
  if (!d || guarded(nullptr, 0, [&] { c = d->s->cache(attn, inst); }) != 0) return nullptr;
  return reinterpret_cast<xtg_hip_kv*>(c);
}

size_t xtg_hip_x_operand_bytes(int k) { return k > 0 ? xtg::hip::Backend::op_bytes(k) : 0; }

int xtg_hip_prep_x(xtg_hip* h, const void* x, int x_dtype, int m, int k, void* op, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "prep_x: NULL handle");
    h->b->prep_x(x, x_dtype, m, k, op);
  });
}

int xtg_hip_matmul_nvfp4_op(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const void* op, int m, float* y, size_t y_offset,
                            char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && ws, "matmul: NULL argument");
    h->b->matmul_op(ws, n_w, op, m, y, y_offset);
  });
}

int xtg_hip_alloc(xtg_hip* h, size_t bytes, void** out, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && out, "alloc: NULL argument");
    *out = h->b->alloc(bytes);
  });
}

void xtg_hip_release(xtg_hip* h, void* mem) {
  if (h) guarded(nullptr, 0, [&] { h->b->release(mem); });
}

int xtg_hip_write(xtg_hip* h, void* mem, size_t offset, const void* src, size_t bytes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && mem && (src || !bytes), "write: NULL argument");
    h->b->write(mem, offset, src, bytes);
  });
}

int xtg_hip_read(xtg_hip* h, const void* mem, size_t offset, void* dst, size_t bytes, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && mem && (dst || !bytes), "read: NULL argument");
    h->b->read(mem, offset, dst, bytes);
  });
}

int xtg_hip_copy(xtg_hip* h, const void* src, size_t src_offset, void* dst, size_t dst_offset, size_t bytes, char* err,
                 int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && src && dst, "copy: NULL argument");
    h->b->copy(src, src_offset, dst, dst_offset, bytes);
  });
}

int xtg_hip_graph_begin(xtg_hip* h, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "graph_begin: NULL handle");
    h->b->graph_begin();
  });
}

int xtg_hip_graph_end(xtg_hip* h, const char* name, xtg_hip_graph** out, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && out, "graph_end: NULL argument");
    *out = reinterpret_cast<xtg_hip_graph*>(h->b->graph_end(name ? name : ""));
  });
}

int xtg_hip_graph_launch(xtg_hip* h, xtg_hip_graph* g, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h && g, "graph_launch: NULL argument");
    h->b->graph_launch(reinterpret_cast<hipGraphExec_t>(g));
  });
}

void xtg_hip_graph_destroy(xtg_hip* h, xtg_hip_graph* g) {
  if (h && g) guarded(nullptr, 0, [&] { h->b->graph_destroy(reinterpret_cast<hipGraphExec_t>(g)); });
}

size_t xtg_hip_read_probe_partials(size_t bytes) { return xtg::hip::read_probe_groups(bytes); }

int xtg_hip_read_probe(xtg_hip* h, const void* src, size_t bytes, uint32_t* out, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "read probe: NULL handle");
    h->b->read_probe(src, bytes, out);
  });
}

int xtg_hip_profile(xtg_hip* h, int enable, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "profile: NULL handle");
    h->b->set_profile(enable == 2 ? 2 : enable != 0 ? 1 : 0);
  });
}

int xtg_hip_profile_report(xtg_hip* h, char* out, int out_len) {
  if (!h) return -1;
  std::string s;
  if (guarded(nullptr, 0, [&] { s = h->b->profile_report(); }) != 0) return -1;
  if (out && out_len > 0) std::snprintf(out, size_t(out_len), "%s", s.c_str());
  return int(s.size());
}

int xtg_hip_finish(xtg_hip* h, char* err, int err_len) {
  return guarded(err, err_len, [&] {
    XTG_CHECK(h, "finish: NULL handle");
    h->b->finish();
  });
}

}  // extern "C"
