#include "backend.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "common.hpp"

namespace xtg::hip {

Backend::Backend(int device) : device_(device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  XTG_CHECK(device >= 0 && device < count, "no HIP device %d (%d present)", device, count);
  HIP_CHECK(hipSetDevice(device));
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  attn_scratch_ = attn_scratch_ptr(device);   // with the device current, once per device
  const std::vector<float2> ident(128, make_float2(1.f, 0.f));   // head_dim up to 256
  HIP_CHECK(hipMalloc(&ident_rope_, ident.size() * sizeof(float2)));
  HIP_CHECK(hipMemcpy(ident_rope_, ident.data(), ident.size() * sizeof(float2), hipMemcpyHostToDevice));
}

Backend::~Backend() {
  // teardown: errors cannot be reported from a destructor; every release is still attempted
  (void)hipSetDevice(device_);
  attn_scratch_let_go(device_, this);
  if (capturing_) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream_, &g);
    if (g) (void)hipGraphDestroy(g);
  }
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& kv : graphs_) (void)hipGraphExecDestroy(kv.first);
  for (auto& kv : weights_) (void)hipFree(kv.second.tiles);
  for (auto& kv : bf16_weights_) (void)hipFree(kv.second.tiles);
  for (void* p : allocs_) (void)hipFree(p);
  for (void* p : {op_, opb_, hx_, hy_, part_, kproc_, stage_, sample_, static_cast<void*>(ident_rope_)})
    if (p) (void)hipFree(p);
  for (void* p : retired_) (void)hipFree(p);
  for (DevKv* c : kvs_) {
    for (void* p : {c->k, c->v, static_cast<void*>(c->kscale), static_cast<void*>(c->vscale),
                    static_cast<void*>(c->slot_pos)})
      if (p) (void)hipFree(p);
    delete c;
  }
  for (auto& f : inv_freq_) (void)hipFree(f.second);
  for (auto& t : rope_) (void)hipFree(t.p);
  for (const Pending& p : pending_) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  for (hipEvent_t e : free_events_) (void)hipEventDestroy(e);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void Backend::ensure(void*& buf, size_t& size, size_t need) {
  if (size >= need) return;
  XTG_CHECK(!capturing_, "scratch of %zu bytes needed during graph capture (run the calls once before capturing)",
            need);
  if (buf) {
    dev_free(buf);   // queued work, or a graph, may still read the old buffer
    buf = nullptr;
    size = 0;
  }
  HIP_CHECK(hipMalloc(&buf, need));
  size = need;
}

void Backend::dev_free(void* p) {
  if (!p) return;
  if (!graphs_.empty()) {
    retired_.push_back(p);
    return;
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipFree(p));
}

void Backend::hold(const void* key, bool owned) {
  XTG_CHECK(weights_.count(static_cast<const uint8_t*>(key)) || bf16_weights_.count(static_cast<const uint16_t*>(key)),
            "hold: no weight prepared for %p", key);
  Hold& h = holds_[key];
  h.count += 1;
  h.owned = h.owned || owned;
}

void Backend::unhold(const void* key) {
  auto it = holds_.find(key);
  if (it == holds_.end()) return;
  if (--it->second.count > 0) return;
  const bool owned = it->second.owned;
  holds_.erase(it);
  if (owned) drop_weight(key);
}

void Backend::drop_weight(const void* key) {
  auto it = weights_.find(static_cast<const uint8_t*>(key));
  if (it != weights_.end()) {
    dev_free(it->second.tiles);
    weight_bytes_ -= it->second.bytes;
    weights_.erase(it);
    return;
  }
  auto jt = bf16_weights_.find(static_cast<const uint16_t*>(key));
  if (jt != bf16_weights_.end()) {
    dev_free(jt->second.tiles);
    weight_bytes_ -= jt->second.bytes;
    bf16_weights_.erase(jt);
  }
}

const PackedNvfp4& Backend::prepare(const xtg_nvfp4& w) {
  XTG_CHECK(w.codes && w.scales, "prepare: NULL codes or scales");
  auto it = weights_.find(w.codes);
  if (it != weights_.end()) {
    XTG_CHECK(it->second.n == w.n_out && it->second.k == w.k, "prepare: weight %p seen before as %dx%d, now %dx%d",
              static_cast<const void*>(w.codes), it->second.n, it->second.k, w.n_out, w.k);
    return it->second;
  }
  XTG_CHECK(w.n_out > 0 && w.k > 0 && w.k % 16 == 0, "prepare: invalid NVFP4 shape %dx%d (k %% 16 == 0)", w.n_out, w.k);
  XTG_CHECK(!capturing_, "prepare: weights must be prepared before a graph capture");
  PackedNvfp4 p;
  p.n = w.n_out;
  p.k = w.k;
  p.nb = (w.n_out + kTileRows - 1) / kTileRows;
  p.kt = (w.k + kTileK - 1) / kTileK;
  p.global = w.global;
  p.bytes = size_t(p.nb) * size_t(p.kt) * kTileBytes;
  // the checkpoint's arrays as they are to a staging buffer (at most kStageBytes: row-blocks at a time), then the
  // tile layout of those row-blocks on the device
  HIP_CHECK(hipMalloc(&p.tiles, p.bytes));
  const size_t row_c = size_t(w.k / 2), row_s = size_t(w.k / 16);
  const int chunk = int(std::max<size_t>(1, kStageBytes / ((row_c + row_s) * kTileRows)) * kTileRows);
  ensure(stage_, stage_size_, size_t(std::min(chunk, p.nb * kTileRows)) * (row_c + row_s) + 256);
  uint8_t* st = static_cast<uint8_t*>(stage_);
  for (int r0 = 0; r0 < w.n_out; r0 += chunk) {
    const int rows = std::min(chunk, w.n_out - r0);
    const size_t cb = size_t(rows) * row_c, s_off = (cb + 255) / 256 * 256;
    HIP_CHECK(hipMemcpyAsync(st, w.codes + size_t(r0) * row_c, cb, hipMemcpyHostToDevice, stream_));
    HIP_CHECK(hipMemcpyAsync(st + s_off, w.scales + size_t(r0) * row_s, size_t(rows) * row_s, hipMemcpyHostToDevice,
                             stream_));
    timed([&] {
      return launch_pack_nvfp4(st, st + s_off, rows, w.k, p.tiles + size_t(r0 / kTileRows) * p.kt * kTileBytes,
                               stream_);
    });
    HIP_CHECK(hipStreamSynchronize(stream_));   // the staging buffer takes the next chunk
  }
  weight_bytes_ += p.bytes;
  return weights_.emplace(w.codes, p).first->second;
}

void Backend::read_tiles(const uint8_t* codes, void* out, size_t bytes) {
  auto it = weights_.find(codes);
  XTG_CHECK(it != weights_.end(), "nvfp4_tiles: no weight prepared for %p", static_cast<const void*>(codes));
  XTG_CHECK(bytes == it->second.bytes, "nvfp4_tiles: %zu bytes for tiles of %zu", bytes, it->second.bytes);
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipMemcpy(out, it->second.tiles, bytes, hipMemcpyDeviceToHost));
}

void Backend::release_weight(const uint8_t* codes) {
  XTG_CHECK(!capturing_, "release_nvfp4: not during a graph capture");
  XTG_CHECK(!holds_.count(codes), "release_nvfp4: weight %p is in use by a Dory session",
            static_cast<const void*>(codes));
  drop_weight(codes);
}

void Backend::matmul_dev(const xtg_nvfp4* ws, int nw, const void* x, int x_dtype, int m, float* y, size_t y_off) {
  XTG_CHECK(nw >= 1 && nw <= 4, "matmul: %d weights (1..4 per call)", nw);
  const int k = ws[0].k;
  XTG_CHECK(m >= 1 && m <= kMaxDeviceRows, "matmul: %d rows (1..%d per device call)", m, kMaxDeviceRows);
  XTG_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0, "matmul: rows at %p are not 16-byte aligned", x);
  if (m <= kMaxRows) {   // the GEMV takes the rows as they are when its shape allows
    XTG_CHECK(x_dtype == kXF32 || x_dtype == kXBF16, "matmul: unknown activation type %d", x_dtype);
    XTG_CHECK(x && y, "matmul: NULL input or output");
    GemvCall c;
    c.nw = nw;
    size_t off = y_off;
    for (int i = 0; i < nw; ++i) {
      XTG_CHECK(ws[i].k == k, "matmul: input widths differ (%d, %d)", ws[i].k, k);
      c.w[i] = &prepare(ws[i]);
      c.y_off[i] = off;
      off += size_t(m) * size_t(ws[i].n_out);
    }
    c.y = y;
    c.m = m;
    c.x = x;
    c.x_dtype = x_dtype;
    c.k = k;
    if (gemv_takes_raw(c)) {
      timed([&] { return launch_gemv(c, stream_); });
      return;
    }
  }
  ensure(op_, op_size_, size_t((m + kMaxRows - 1) / kMaxRows) * op_bytes(k));
  prep_x(x, x_dtype, m, k, op_);
  matmul_op(ws, nw, op_, m, y, y_off);
}

void Backend::prep_x(const void* x, int x_dtype, int m, int k, void* op, float* copy) {
  XTG_CHECK(m >= 1 && m <= kMaxDeviceRows, "matmul: %d rows (1..%d per device call)", m, kMaxDeviceRows);
  XTG_CHECK(x_dtype == kXF32 || x_dtype == kXBF16, "matmul: unknown activation type %d", x_dtype);
  XTG_CHECK(x && op, "prep_x: NULL input or operand");
  XTG_CHECK(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(op) % 16 == 0,
            "prep_x: rows and operand must be 16-byte aligned");
  timed([&] { return launch_prep_x(x, x_dtype, m, k, op, stream_, copy); });
}

int Backend::matmul_op(const xtg_nvfp4* ws, int nw, const void* op, int m, float* y, size_t y_off,
                       const float* col_scale, int ksplit) {
  XTG_CHECK(ksplit == 1 || ksplit == 2, "matmul: a K split in %d parts (1 or 2)", ksplit);
  XTG_CHECK(nw >= 1 && nw <= 4, "matmul: %d weights (1..4 per call)", nw);
  XTG_CHECK(!col_scale || nw == 1, "matmul: a column scale applies to a single weight");
  XTG_CHECK(m >= 1 && m <= kMaxDeviceRows, "matmul: %d rows (1..%d per device call)", m, kMaxDeviceRows);
  XTG_CHECK(op && y, "matmul: NULL operand or output");
  const int k = ws[0].k;
  GemvCall c;
  c.nw = nw;
  size_t off = y_off;
  for (int i = 0; i < nw; ++i) {
    XTG_CHECK(ws[i].k == k, "matmul: input widths differ (%d, %d)", ws[i].k, k);
    c.w[i] = &prepare(ws[i]);
    c.y_off[i] = off;
    off += size_t(m) * size_t(ws[i].n_out);
  }
  c.y = y;
  c.m = m;
  c.xop = op;
  c.xinv = reinterpret_cast<const float*>(static_cast<const char*>(op) + xop_bytes(k));
  c.col_scale[0] = col_scale;
  // up to 8 rows: the bandwidth-bound GEMV; more (a prefill chunk): the matrix-core GEMM over 8-row groups
  if (m > kMaxRows) {
    timed([&] { return launch_gemm(c, stream_); });
    return 1;
  }
  if (ksplit == 2 && m >= 2) {
    c.ksplit = 2;
    c.y_part = off - y_off;   // one output set: m rows of every weight
  }
  timed([&] { return launch_gemv(c, stream_); });
  return c.ksplit;
}

void Backend::read_probe(const void* src, size_t bytes, uint32_t* out) {
  timed([&] { return launch_read_probe(src, bytes, out, stream_); });
}

int Backend::matmul_fused(const xtg_nvfp4* ws, int nw, FusedGemv f, const void* op, int m, float* y) {
  XTG_CHECK(nw >= 1 && nw <= 4, "matmul: %d weights (1..4 per call)", nw);
  XTG_CHECK(m == 1, "fused matmul: %d rows (one)", m);
  XTG_CHECK(y, "matmul: NULL output");
  if (f.in == kInOp && f.out == kOutPlain) {   // nothing rides on it: the plain GEMV
    matmul_op(ws, nw, op, m, y, 0);
    return 0;
  }
  const int k = ws[0].k;
  GemvCall& c = f.c;
  c.nw = nw;
  size_t off = 0;
  for (int i = 0; i < nw; ++i) {
    XTG_CHECK(ws[i].k == k, "matmul: input widths differ (%d, %d)", ws[i].k, k);
    c.w[i] = &prepare(ws[i]);
    c.y_off[i] = off;
    if (f.out != kOutSwiglu) off += size_t(m) * size_t(ws[i].n_out);
  }
  c.y = y;
  c.m = m;
  c.k = k;
  if (f.in == kInOp) {
    XTG_CHECK(op, "fused matmul: no operand");
    c.xop = op;
    c.xinv = reinterpret_cast<const float*>(static_cast<const char*>(op) + xop_bytes(k));
  } else if (f.in == kInSlerp) {
    XTG_CHECK(op, "fused matmul: no operand");
    c.xop = op;   // the producer's linear-form operand, its factors in f.in_ia / f.in_ib
  }
  timed([&] { return launch_gemv_fused(f, stream_); });
  return fused_gemv_groups(f);
}

// ------------------------------------------------------------------------------------------------ BF16 path

const PackedBf16& Backend::prepare(const xtg_bf16& w) {
  XTG_CHECK(w.data, "prepare_bf16: NULL data");
  auto it = bf16_weights_.find(w.data);
  if (it != bf16_weights_.end()) {
    XTG_CHECK(it->second.n == w.n_out && it->second.k == w.k,
              "prepare_bf16: weight %p seen before as %dx%d, now %dx%d", static_cast<const void*>(w.data),
              it->second.n, it->second.k, w.n_out, w.k);
    return it->second;
  }
  XTG_CHECK(w.n_out > 0 && w.k > 0 && w.k % 4 == 0, "prepare_bf16: invalid BF16 shape %dx%d (k %% 4 == 0)", w.n_out,
            w.k);
  XTG_CHECK(!capturing_, "prepare_bf16: weights must be prepared before a graph capture");
  std::vector<uint16_t> host;
  pack_bf16_tiles(w.data, w.n_out, w.k, host);
  PackedBf16 p;
  p.n = w.n_out;
  p.k = w.k;
  p.nb = (w.n_out + kTileRows - 1) / kTileRows;
  p.kt = (w.k + kTileK - 1) / kTileK;
  p.bytes = host.size() * sizeof(uint16_t);
  HIP_CHECK(hipMalloc(&p.tiles, p.bytes));
  const hipError_t e = hipMemcpy(p.tiles, host.data(), p.bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(p.tiles);
    HIP_CHECK(e);
  }
  weight_bytes_ += p.bytes;
  return bf16_weights_.emplace(w.data, p).first->second;
}

void Backend::release_bf16(const uint16_t* data) {
  XTG_CHECK(!capturing_, "release_bf16: not during a graph capture");
  XTG_CHECK(!holds_.count(data), "release_bf16: weight %p is in use by a Dory session", static_cast<const void*>(data));
  drop_weight(data);
}

void Backend::matmul_bf16_dev(const xtg_bf16& w, const void* x, int x_dtype, int m, float* y, size_t y_off,
                              const float* col_scale) {
  XTG_CHECK(m >= 1 && m <= kMaxRows, "matmul_bf16: %d rows (1..%d per device call)", m, kMaxRows);
  XTG_CHECK(x_dtype == kXF32 || x_dtype == kXBF16, "matmul_bf16: unknown activation type %d", x_dtype);
  XTG_CHECK(x && y, "matmul_bf16: NULL input or output");
  const PackedBf16& p = prepare(w);
  ensure(opb_, opb_size_, xop_bf16_bytes(w.k));
  timed([&] { return launch_prep_x_bf16(x, x_dtype, m, w.k, opb_, stream_); });
  timed([&] { return launch_gemv_bf16(p, opb_, m, y + y_off, col_scale, stream_); });
}

void Backend::matmul_bf16(const xtg_bf16& w, const float* x, int m, float* y) {
  XTG_CHECK(m >= 1 && x && y, "matmul_bf16: %d rows", m);
  XTG_CHECK(!capturing_, "matmul_bf16: the host-synchronous call cannot be captured (use the device call)");
  prepare(w);
  ensure(hx_, hx_size_, size_t(kMaxRows) * size_t(w.k) * sizeof(float));
  ensure(hy_, hy_size_, size_t(kMaxRows) * size_t(w.n_out) * sizeof(float));
  for (int r0 = 0; r0 < m; r0 += kMaxRows) {
    const int rows = std::min(kMaxRows, m - r0);
    HIP_CHECK(hipMemcpyAsync(hx_, x + size_t(r0) * size_t(w.k), size_t(rows) * size_t(w.k) * sizeof(float),
                             hipMemcpyHostToDevice, stream_));
    matmul_bf16_dev(w, hx_, kXF32, rows, static_cast<float*>(hy_), 0);
    HIP_CHECK(hipMemcpyAsync(y + size_t(r0) * size_t(w.n_out), hy_, size_t(rows) * size_t(w.n_out) * sizeof(float),
                             hipMemcpyDeviceToHost, stream_));
    HIP_CHECK(hipStreamSynchronize(stream_));
  }
}

// ------------------------------------------------------------------------------------------------- KV caches

DevKv* Backend::kv_create(int kv_heads, int head_dim, long long slots, int ring, int dtype) {
  XTG_CHECK(!capturing_, "kv_create: not during a graph capture");
  XTG_CHECK(dtype == XTG_KV_BF16 || dtype == XTG_KV_FP8, "kv_create: unknown KV dtype %d", dtype);
  XTG_CHECK(head_dim == 64 || head_dim == 128 || head_dim == 256, "kv_create: head_dim %d (64, 128 or 256)",
            head_dim);
  XTG_CHECK(kv_heads > 0, "kv_create: %d KV heads", kv_heads);
  const long long n = ring > 0 ? ring : slots;   // kv.cpp:42-44: ring > 0 gives a ring of `ring` slots
  XTG_CHECK(n > 0 && n < (1LL << 30), "kv_create: %lld slots", n);
  auto c = std::make_unique<DevKv>();
  c->kv_heads = kv_heads;
  c->head_dim = head_dim;
  c->slots = n;
  c->slots_pad = int((n + 31) / 32 * 32);
  c->ring = ring > 0;
  c->fp8 = dtype == XTG_KV_FP8;
  try {
    HIP_CHECK(hipMalloc(&c->k, c->data_bytes()));
    HIP_CHECK(hipMalloc(&c->v, c->data_bytes()));
    HIP_CHECK(hipMalloc(&c->slot_pos, size_t(c->slots_pad) * sizeof(int)));
    if (c->fp8) {
      HIP_CHECK(hipMalloc(&c->kscale, c->scale_bytes()));
      HIP_CHECK(hipMalloc(&c->vscale, c->scale_bytes()));
    }
  } catch (...) {
    for (void* p : {c->k, c->v, static_cast<void*>(c->kscale), static_cast<void*>(c->vscale),
                    static_cast<void*>(c->slot_pos)})
      if (p) (void)hipFree(p);
    throw;
  }
  DevKv* p = c.release();
  kvs_.insert(p);
  clear_kv(p);
  return p;
}

// Every slot empty: zero codes and scales, slot positions -1.
void Backend::clear_kv(DevKv* c) {
  HIP_CHECK(hipMemsetAsync(c->k, 0, c->data_bytes(), stream_));
  HIP_CHECK(hipMemsetAsync(c->v, 0, c->data_bytes(), stream_));
  if (c->fp8) {
    HIP_CHECK(hipMemsetAsync(c->kscale, 0, c->scale_bytes(), stream_));
    HIP_CHECK(hipMemsetAsync(c->vscale, 0, c->scale_bytes(), stream_));
  }
  HIP_CHECK(hipMemsetAsync(c->slot_pos, 0xff, size_t(c->slots_pad) * sizeof(int), stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::kv_destroy(DevKv* c) {
  auto it = kvs_.find(c);
  if (it == kvs_.end()) return;
  XTG_CHECK(!capturing_, "kv_destroy: not during a graph capture");
  for (void* p : {c->k, c->v, static_cast<void*>(c->kscale), static_cast<void*>(c->vscale),
                  static_cast<void*>(c->slot_pos)})
    dev_free(p);
  kvs_.erase(it);
  delete c;
}

void Backend::kv_store(DevKv* c, long long pos, int n, const float* k, const float* v) {
  XTG_CHECK(kvs_.count(c), "kv_store: unknown cache");
  XTG_CHECK(n >= 0 && pos >= 0, "kv_store: %d rows at %lld", n, pos);
  // kv.cpp:78: a linear cache holds positions below its capacity
  XTG_CHECK(c->ring || pos + n <= c->slots, "KV cache full: position %lld of %lld", pos + n, c->slots);
  XTG_CHECK(pos + n < (1LL << 31), "kv_store: position %lld beyond the 32-bit slot positions", pos + n);
  if (n == 0) return;
  XTG_CHECK(k && v, "kv_store: NULL rows");
  timed([&] { return launch_kv_store(*c, pos, n, k, v, stream_); });
}

namespace {

// The value of an E4M3 code (engine/src/fp.cpp:12-28: bias 7, subnormal step 2^-9, 0x7f / 0xff NaN).
float e4m3_value(uint8_t b) {
  const int e = (b >> 3) & 15, m = b & 7;
  float mag;
  if ((b & 0x7f) == 0x7f)
    mag = NAN;
  else if (e == 0)
    mag = std::ldexp(float(m), -9);
  else
    mag = std::ldexp(1.f + float(m) / 8.f, e - 7);
  return (b & 0x80) ? -mag : mag;
}

}  // namespace

void Backend::kv_load(const DevKv* c, int h, long long p0, long long p1, float* k, float* v) {
  XTG_CHECK(kvs_.count(const_cast<DevKv*>(c)), "kv_load: unknown cache");
  XTG_CHECK(!capturing_, "kv_load: not during a graph capture");
  XTG_CHECK(h >= 0 && h < c->kv_heads && p0 >= 0 && p0 <= p1, "kv_load: head %d, positions %lld..%lld", h, p0, p1);
  XTG_CHECK(c->ring || p1 <= c->slots, "kv_load: position %lld beyond the cache", p1);
  const int d = c->head_dim;
  std::vector<uint8_t> snap(kv_bytes(c));
  snapshot(c, snap.data());
  const uint8_t* hk = snap.data();
  const uint8_t* hv = hk + c->data_bytes();
  const float* ks = reinterpret_cast<const float*>(hv + c->data_bytes());
  const float* vs = ks + size_t(c->kv_heads) * size_t(c->slots_pad);
  for (long long p = p0; p < p1; ++p) {
    const int slot = int(c->ring ? p % c->slots : p);
    float* ok = k + size_t(p - p0) * size_t(d);
    float* ov = v + size_t(p - p0) * size_t(d);
    if (c->fp8) {
      const size_t si = size_t(h) * size_t(c->slots_pad) + size_t(slot);
      for (int j = 0; j < d; ++j) {   // kv.cpp:128-136: code value times the row's scale
        ok[j] = e4m3_value(hk[kv_k8_index(h, slot, j, c->slots_pad, d)]) * ks[si];
        ov[j] = e4m3_value(hv[kv_v8_index(h, slot, j, c->slots_pad, d)]) * vs[si];
      }
    } else {
      const uint16_t* bk = reinterpret_cast<const uint16_t*>(hk);
      const uint16_t* bv = reinterpret_cast<const uint16_t*>(hv);
      for (int j = 0; j < d; ++j) {
        const uint32_t kb = uint32_t(bk[kv_k_index(h, slot, j, c->slots_pad, d)]) << 16;
        const uint32_t vb = uint32_t(bv[kv_v_index(h, slot, j, c->slots_pad, d)]) << 16;
        std::memcpy(ok + j, &kb, 4);
        std::memcpy(ov + j, &vb, 4);
      }
    }
  }
}

// Snapshot layout: K data, V data, K scales, V scales (FP8 only), slot positions, each in its device layout.
size_t Backend::kv_bytes(const DevKv* c) const {
  return 2 * c->data_bytes() + 2 * c->scale_bytes() + size_t(c->slots_pad) * sizeof(int);
}

void Backend::snapshot(const DevKv* c, void* out) {
  char* o = static_cast<char*>(out);
  const size_t db = c->data_bytes(), sb = c->scale_bytes();
  HIP_CHECK(hipMemcpyAsync(o, c->k, db, hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipMemcpyAsync(o + db, c->v, db, hipMemcpyDeviceToHost, stream_));
  if (sb) {
    HIP_CHECK(hipMemcpyAsync(o + 2 * db, c->kscale, sb, hipMemcpyDeviceToHost, stream_));
    HIP_CHECK(hipMemcpyAsync(o + 2 * db + sb, c->vscale, sb, hipMemcpyDeviceToHost, stream_));
  }
  HIP_CHECK(hipMemcpyAsync(o + 2 * db + 2 * sb, c->slot_pos, size_t(c->slots_pad) * sizeof(int),
                           hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::kv_save(const DevKv* c, void* out, size_t bytes) {
  XTG_CHECK(kvs_.count(const_cast<DevKv*>(c)), "kv_save: unknown cache");
  XTG_CHECK(!capturing_, "kv_save: not during a graph capture");
  XTG_CHECK(bytes == kv_bytes(c), "kv_save: %zu bytes for a cache of %zu", bytes, kv_bytes(c));
  snapshot(c, out);
}

void Backend::kv_restore(DevKv* c, const void* in, size_t bytes) {
  XTG_CHECK(kvs_.count(c), "kv_restore: unknown cache");
  XTG_CHECK(!capturing_, "kv_restore: not during a graph capture");
  XTG_CHECK(bytes == kv_bytes(c), "KV snapshot of %zu bytes for a cache of %zu", bytes, kv_bytes(c));
  const char* s = static_cast<const char*>(in);
  const size_t db = c->data_bytes(), sb = c->scale_bytes();
  HIP_CHECK(hipMemcpyAsync(c->k, s, db, hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(c->v, s + db, db, hipMemcpyHostToDevice, stream_));
  if (sb) {
    HIP_CHECK(hipMemcpyAsync(c->kscale, s + 2 * db, sb, hipMemcpyHostToDevice, stream_));
    HIP_CHECK(hipMemcpyAsync(c->vscale, s + 2 * db + sb, sb, hipMemcpyHostToDevice, stream_));
  }
  HIP_CHECK(hipMemcpyAsync(c->slot_pos, s + 2 * db + 2 * sb, size_t(c->slots_pad) * sizeof(int),
                           hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::kv_release(DevKv* c) {
  XTG_CHECK(kvs_.count(c), "kv_release: unknown cache");
  XTG_CHECK(!capturing_, "kv_release: not during a graph capture");
  clear_kv(c);
}

void Backend::kv_copy(const DevKv* src, DevKv* dst) {
  XTG_CHECK(kvs_.count(const_cast<DevKv*>(src)) && kvs_.count(dst), "kv_copy: unknown cache");
  XTG_CHECK(src->kv_heads == dst->kv_heads && src->head_dim == dst->head_dim && src->slots == dst->slots &&
                src->ring == dst->ring && src->fp8 == dst->fp8,
            "kv_copy: caches of different shapes or dtypes");
  if (src == dst) return;
  HIP_CHECK(hipMemcpyAsync(dst->k, src->k, src->data_bytes(), hipMemcpyDeviceToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(dst->v, src->v, src->data_bytes(), hipMemcpyDeviceToDevice, stream_));
  if (src->fp8) {
    HIP_CHECK(hipMemcpyAsync(dst->kscale, src->kscale, src->scale_bytes(), hipMemcpyDeviceToDevice, stream_));
    HIP_CHECK(hipMemcpyAsync(dst->vscale, src->vscale, src->scale_bytes(), hipMemcpyDeviceToDevice, stream_));
  }
  HIP_CHECK(hipMemcpyAsync(dst->slot_pos, src->slot_pos, size_t(src->slots_pad) * sizeof(int),
                           hipMemcpyDeviceToDevice, stream_));
}

void Backend::check_attention(const DevKv* c, int n_q, long long pos0, const float* q, const float* k, const float* v,
                              const float* out) const {
  XTG_CHECK(kvs_.count(const_cast<DevKv*>(c)), "attention: unknown cache");
  XTG_CHECK(n_q >= 1 && pos0 >= 0, "attention: %d rows at %lld", n_q, pos0);
  XTG_CHECK(q && k && v && out, "attention: NULL argument");
  for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(k), static_cast<const void*>(v),
                        static_cast<const void*>(out)})
    XTG_CHECK(reinterpret_cast<uintptr_t>(p) % 16 == 0, "attention: arguments must be 16-byte aligned");
}

void Backend::attention_noalloc(const DevKv* c, int n_q, long long pos0, int heads, int window, float scale,
                                const float* q, const float* k, const float* v, float* out) {
  check_attention(c, n_q, pos0, q, k, v, out);
  const AttnPlan p = attn_plan(*c, n_q, heads, pos0, window);
  const size_t need = p.part_floats() * sizeof(float);
  XTG_CHECK(need <= kAttnScratchBytes,
            "attention_noalloc: %d rows over %d KV heads (%d key splits) need %zu bytes of partials; the fixed scratch "
            "holds %zu",
            n_q, c->kv_heads, p.splits, need, kAttnScratchBytes);
  XTG_CHECK(attn_scratch_claim(device_, this),
            "attention_noalloc: another open backend on device %d uses the device's fixed scratch (calls from two "
            "backends would race on it); close that backend first",
            device_);
  attention_launches(c, p, n_q, pos0, heads, window, scale, q, k, v, out, static_cast<float*>(attn_scratch_));
}

void Backend::attention_launches(const DevKv* c, const AttnPlan& p, int n_q, long long pos0, int heads, int window,
                                 float scale, const float* q, const float* k, const float* v, float* out,
                                 float* part) {
  if (attn_step_fuses(p, n_q) && !std::getenv("XTG_ATTN_UNFUSED")) {
    // the producer's work-groups take the own keys from q and k as they are (write_q off: q is only read)
    timed([&] {
      return launch_attn_step(*c, p, const_cast<float*>(q), k, v, nullptr, n_q, heads, pos0, window, scale,
                              ident_rope_, nullptr, false, part, stream_, true);
    });
    timed([&] { return launch_attn_merge_heads(p, n_q, heads, part, out, stream_); });
    return;
  }
  timed([&] { return launch_attn_own(p, 0, p.blocks, q, k, v, n_q, heads, window, scale, part, stream_); });
  if (p.splits > 0)
    timed([&] { return launch_attn_scan(*c, p, 0, p.blocks, q, n_q, heads, pos0, window, scale, part, stream_); });
  timed([&] { return launch_attn_merge(p, n_q, heads, part, out, stream_); });
}

void Backend::attention(const DevKv* c, int n_q, long long pos0, int heads, int window, float scale, const float* q,
                        const float* k, const float* v, float* out) {
  check_attention(c, n_q, pos0, q, k, v, out);
  const AttnPlan p = attn_plan(*c, n_q, heads, pos0, window);
  ensure(part_, part_size_, p.part_floats() * sizeof(float));
  // every row block in one launch each (the last block may be partial: its q-cols past the rows are masked)
  attention_launches(c, p, n_q, pos0, heads, window, scale, q, k, v, out, static_cast<float*>(part_));
}

void Backend::attn_step(DevKv* c, int m, long long pos0, int heads, int window, float scale, float theta, float* q,
                        float* k, const float* v, const float* qscale, const float* g, const float* gscale,
                        float* out, void* op, bool store, float* gate_rec) {
  XTG_CHECK(kvs_.count(c), "attention step: unknown cache");
  XTG_CHECK(!gate_rec || (m == 1 && out && !op), "attention step: the gate's records take one row, out and no operand");
  XTG_CHECK(m >= 1 && pos0 >= 0, "attention step: %d rows at %lld", m, pos0);
  XTG_CHECK(pos0 + m < (1LL << 31), "attention step: position %lld beyond the 32-bit slot positions", pos0 + m);
  XTG_CHECK(c->ring || pos0 + m <= c->slots, "attention step: context full (%lld + %d > %lld slots)", pos0, m,
            c->slots);
  XTG_CHECK(q && k && v && g && gscale, "attention step: NULL argument");
  const AttnPlan p = attn_plan(*c, m, heads, pos0, window);
  ensure(part_, part_size_, p.part_floats() * sizeof(float));
  float* part = static_cast<float*>(part_);
  if (m > kProdRows) {
    const float* f = inv_freq(theta, c->head_dim);
    // a prefill chunk (the reference's order, dory.cpp:481-515): RoPE + norms in place, the attention over the
    // read-only cache and the chunk's own keys (matrix-core own-key tiles), the store of the chunk's k / v, then
    // the merge with the gate and norm
    timed([&] { return launch_qk_rope_norm(q, k, m, heads, c->kv_heads, c->head_dim, pos0, f,
                                           qscale, stream_); });
    timed([&] { return launch_attn_own(p, 0, p.blocks, q, k, v, m, heads, window, scale, part, stream_); });
    if (p.splits > 0)
      timed([&] { return launch_attn_scan(*c, p, 0, p.blocks, q, m, heads, pos0, window, scale, part, stream_); });
    if (store) timed([&] { return launch_kv_store(*c, pos0, m, k, v, stream_); });
    timed([&] { return launch_attn_gate(p, m, heads, part, g, gscale, out, op, stream_); });
    return;
  }
  // storing before the scan hides nothing the scan should see: a linear cache's new slots are masked as
  // positions >= pos0, and a ring of window + m - 1 slots or more only drops positions outside every row's window
  const bool store_first = store && (!c->ring || (window > 0 && c->slots >= (long long)window + m - 1));
  float* kout = nullptr;   // the processed k rows, for a store after the scan
  if (store && !store_first) {
    ensure(kproc_, kproc_size_, size_t(m) * size_t(c->kv_heads) * size_t(c->head_dim) * sizeof(float));
    kout = static_cast<float*>(kproc_);
  }
  const float2* rt = rope_table(theta, c->head_dim, pos0 + m);
  if (attn_step_fuses(p, m) && !std::getenv("XTG_ATTN_UNFUSED")) {
    timed([&] {
      return launch_attn_step(*c, p, q, k, v, kout, m, heads, pos0, window, scale, rt, qscale, store_first, part,
                              stream_);
    });
  } else {
    timed([&] {
      return launch_qk_produce(*c, p, q, k, v, kout, m, heads, pos0, window, scale, rt, qscale, store_first, part,
                               stream_);
    });
    if (p.splits > 0)
      timed([&] { return launch_attn_scan(*c, p, 0, p.blocks, q, m, heads, pos0, window, scale, part, stream_); });
  }
  if (store && !store_first) timed([&] { return launch_kv_store(*c, pos0, m, kout, v, stream_); });
  if (gate_rec)
    timed([&] { return launch_attn_gate_heads(p, heads, part, g, gscale, out, gate_rec, stream_); });
  else
    timed([&] { return launch_attn_gate(p, m, heads, part, g, gscale, out, op, stream_); });
}

// ---------------------------------------------------------------------------------------------- row kernels

const float* Backend::inv_freq(float theta, int d) {
  for (auto& f : inv_freq_)
    if (f.first.first == theta && f.first.second == d) return f.second;
  XTG_CHECK(!capturing_, "rope: the table for theta %g, head_dim %d must exist before a graph capture", theta, d);
  std::vector<float> h(size_t(d / 2));
  for (int i = 0; i < d / 2; ++i) h[size_t(i)] = 1.f / std::pow(theta, float(2 * i) / float(d));
  float* p = nullptr;
  HIP_CHECK(hipMalloc(&p, h.size() * sizeof(float)));
  HIP_CHECK(hipMemcpy(p, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
  inv_freq_.push_back({{theta, d}, p});
  return p;
}

const float2* Backend::rope_table(float theta, int d, long long n_pos) {
  XTG_CHECK(n_pos > 0 && n_pos <= (1LL << 31), "rope: a table of %lld positions", n_pos);
  RopeTable* t = nullptr;
  for (auto& r : rope_)
    if (r.theta == theta && r.d == d) t = &r;
  if (t && t->n >= n_pos) return t->p;
  XTG_CHECK(!capturing_, "rope: the table for theta %g, head_dim %d must cover position %lld before a graph capture",
            theta, d, n_pos - 1);
  const float* f = inv_freq(theta, d);
  const long long n = std::min(std::max({n_pos, t ? 2 * t->n : 0LL, 4096LL}), 1LL << 31);
  float2* p = nullptr;
  HIP_CHECK(hipMalloc(&p, size_t(n) * size_t(d / 2) * sizeof(float2)));
  timed([&] { return launch_rope_table(f, d, n, p, stream_); });
  if (t) {
    dev_free(t->p);
    t->p = p;
    t->n = n;
  } else {
    rope_.push_back({theta, d, n, p});
  }
  return p;
}

void Backend::qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0, float theta,
                           const float* qscale) {
  XTG_CHECK(q && k && m >= 1, "rope: NULL argument or %d rows", m);
  const float* f = inv_freq(theta, d);
  timed([&] { return launch_qk_rope_norm(q, k, m, heads, kv_heads, d, pos0, f, qscale, stream_); });
}

void Backend::slerp_norm(float* x, const float* o, const float* lr, int rows, int w, void* op, size_t part) {
  XTG_CHECK(x && o && lr && rows >= 1 && w >= 1, "slerp: bad arguments");
  timed([&] { return launch_slerp_norm(x, o, lr, rows, w, op, stream_, part); });
}

void Backend::swiglu_norm(const float* g, const float* u, const float* sg, const float* su, int rows, int w,
                          float* out, void* op, size_t part) {
  XTG_CHECK(g && u && sg && su && rows >= 1 && w >= 1, "swiglu: bad arguments");
  timed([&] { return launch_swiglu_norm(g, u, sg, su, rows, w, out, op, stream_, part); });
}

void Backend::gate_norm(const float* a, const float* gate, const float* gs, int rows, int w, float* out, void* op) {
  XTG_CHECK(a && gate && gs && rows >= 1 && w >= 1, "gate_norm: bad arguments");
  timed([&] { return launch_gate_norm(a, gate, gs, rows, w, out, op, stream_); });
}

void Backend::add_norm(const float* a, const float* b, float* out, int rows, int w, void* op) {
  XTG_CHECK(a && out && rows >= 1 && w >= 1, "add_norm: bad arguments");
  timed([&] { return launch_add_norm(a, b, out, rows, w, op, stream_); });
}

void Backend::argmax(const float* x, int rows, int n, int* out) {
  XTG_CHECK(x && out && rows >= 1 && n >= 1, "argmax: bad arguments");
  if (rows <= kMaxSampleRows && n > 4096) {   // a vocabulary row: over slices, many work-groups a row
    ensure(sample_, sample_size_, sample_scratch_bytes(rows, n));
    timed([&] { return launch_argmax_slices(x, rows, n, out, sample_, stream_); });
    return;
  }
  timed([&] { return launch_argmax(x, rows, n, out, stream_); });
}

void Backend::sample(const float* x, int rows, int n, float temperature, float top_p, int top_k, float min_p,
                     const double* u, int* out) {
  if (temperature <= 0.f) {   // greedy (sampler.cpp:41): no draw is used
    argmax(x, rows, n, out);
    return;
  }
  XTG_CHECK(x && out && u && rows >= 1 && n >= 1, "sample: bad arguments");
  XTG_CHECK(rows <= kMaxSampleRows, "sample: %d rows (1..%d per call)", rows, kMaxSampleRows);
  ensure(sample_, sample_size_, sample_scratch_bytes(rows, n));
  timed([&] { return launch_sample(x, rows, n, temperature, top_p, top_k, min_p, u, out, sample_, stream_); });
}

hipEvent_t Backend::event() {
  if (!free_events_.empty()) {
    hipEvent_t e = free_events_.back();
    free_events_.pop_back();
    return e;
  }
  hipEvent_t e;
  HIP_CHECK(hipEventCreate(&e));
  return e;
}

void Backend::set_profile(int mode) {
  XTG_CHECK(!capturing_, "profile: not during graph capture");
  XTG_CHECK(mode >= 0 && mode <= 2, "profile: mode %d (0 off, 1 totals, 2 totals and the launch sequence)", mode);
  if (profile_ && mode != profile_) profile_report();   // settle what was recorded
  profile_ = mode;
}

void Backend::graph_begin() {
  XTG_CHECK(!capturing_, "graph_begin: a capture is already open");
  XTG_CHECK(!profile_, "graph_begin: profiling is on (events cannot be timed inside a graph)");
  HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
  capturing_ = true;
}

hipGraphExec_t Backend::graph_end(const std::string& name) {
  XTG_CHECK(capturing_, "graph_end: no capture open");
  capturing_ = false;
  hipGraph_t g = nullptr;
  HIP_CHECK(hipStreamEndCapture(stream_, &g));
  hipGraphExec_t exec = nullptr;
  hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) fail("hipGraphInstantiate failed: %s", hipGetErrorString(e));
  graphs_[exec] = name.empty() ? strf("graph#%zu", graphs_.size()) : name;
  return exec;
}

void Backend::graph_launch(hipGraphExec_t g) {
  auto it = graphs_.find(g);
  XTG_CHECK(it != graphs_.end(), "graph_launch: unknown graph");
  XTG_CHECK(!capturing_, "graph_launch: not during a capture");
  timed([&] {
    HIP_CHECK(hipGraphLaunch(g, stream_));
    return it->second;
  });
}

void Backend::graph_destroy(hipGraphExec_t g) {
  auto it = graphs_.find(g);
  if (it == graphs_.end()) return;
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipGraphExecDestroy(g));
  graphs_.erase(it);
  if (graphs_.empty()) {   // nothing can address the retired memory any more
    std::vector<void*> r;
    r.swap(retired_);
    for (void* p : r) HIP_CHECK(hipFree(p));
  }
}

std::string Backend::profile_report() {
  HIP_CHECK(hipStreamSynchronize(stream_));
  for (const Pending& p : pending_) {
    float ms = 0;
    HIP_CHECK(hipEventElapsedTime(&ms, p.a, p.b));
    auto it = std::find_if(totals_.begin(), totals_.end(), [&](const auto& t) { return t.first == p.name; });
    if (it == totals_.end()) it = totals_.insert(totals_.end(), {p.name, Total{}});
    it->second.calls += 1;
    it->second.ms += ms;
  }
  std::string s = "{\"kernels\": {";
  for (size_t i = 0; i < totals_.size(); ++i)
    s += strf("%s\"%s\": {\"calls\": %ld, \"ms\": %.6f}", i ? ", " : "", totals_[i].first.c_str(),
              totals_[i].second.calls, totals_[i].second.ms);
  s += "}";
  if (profile_ == 2) {   // every launch in queue order
    s += ", \"launches\": [";
    for (size_t i = 0; i < pending_.size(); ++i) {
      float ms = 0;
      HIP_CHECK(hipEventElapsedTime(&ms, pending_[i].a, pending_[i].b));
      s += strf("%s[\"%s\", %.6f]", i ? ", " : "", pending_[i].name.c_str(), ms);
    }
    s += "]";
  }
  s += "}";
  for (const Pending& p : pending_) {
    free_events_.push_back(p.a);
    free_events_.push_back(p.b);
  }
  pending_.clear();
  totals_.clear();
  return s;
}

void Backend::matmul(const xtg_nvfp4* ws, int nw, const float* x, int m, float* const* ys) {
  XTG_CHECK(nw >= 1 && m >= 1 && x, "matmul: %d weights, %d rows", nw, m);
  XTG_CHECK(!capturing_, "matmul: the host-synchronous call cannot be captured (use the device call)");
  const int k = ws[0].k;
  for (int i = 0; i < nw; ++i) XTG_CHECK(ws[i].k == k && k % 16 == 0, "matmul: input widths differ (%d, %d)", ws[i].k, k);
  // more than four weights: groups of four, each group one fused launch
  size_t out_per_row = 0;
  for (int i = 0; i < nw; ++i) out_per_row += size_t(ws[i].n_out);
  const int pass = std::min(m, kHostPassRows);
  ensure(hx_, hx_size_, size_t(pass) * size_t(k) * sizeof(float));
  ensure(hy_, hy_size_, size_t(pass) * out_per_row * sizeof(float));
  for (int r0 = 0; r0 < m; r0 += pass) {
    const int rows = std::min(pass, m - r0);
    HIP_CHECK(hipMemcpyAsync(hx_, x + size_t(r0) * size_t(k), size_t(rows) * size_t(k) * sizeof(float),
                             hipMemcpyHostToDevice, stream_));
    size_t off = 0;
    for (int i0 = 0; i0 < nw; i0 += 4) {
      const int n = std::min(4, nw - i0);
      matmul_dev(ws + i0, n, hx_, kXF32, rows, static_cast<float*>(hy_), off);
      for (int i = i0; i < i0 + n; ++i) off += size_t(rows) * size_t(ws[i].n_out);
    }
    off = 0;
    for (int i = 0; i < nw; ++i) {
      const size_t bytes = size_t(rows) * size_t(ws[i].n_out) * sizeof(float);
      HIP_CHECK(hipMemcpyAsync(ys[i] + size_t(r0) * size_t(ws[i].n_out), static_cast<char*>(hy_) + off * sizeof(float),
                               bytes, hipMemcpyDeviceToHost, stream_));
      off += size_t(rows) * size_t(ws[i].n_out);
    }
    HIP_CHECK(hipStreamSynchronize(stream_));
  }
}

void* Backend::alloc(size_t bytes) {
  void* p = nullptr;
  HIP_CHECK(hipMalloc(&p, std::max<size_t>(bytes, 4)));
  allocs_.insert(p);
  return p;
}

void Backend::release(void* p) {
  if (!p) return;
  XTG_CHECK(!capturing_, "release: not during a graph capture");
  auto it = allocs_.find(p);
  XTG_CHECK(it != allocs_.end(), "release: %p was not allocated by this backend", p);
  allocs_.erase(it);
  dev_free(p);
}

void Backend::write(void* dst, size_t offset, const void* src, size_t bytes) {
  XTG_CHECK(!capturing_, "write: blocking copies cannot be captured");
  if (!bytes) return;
  HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + offset, src, bytes, hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::read(const void* src, size_t offset, void* dst, size_t bytes) {
  XTG_CHECK(!capturing_, "read: blocking copies cannot be captured");
  if (bytes)
    HIP_CHECK(hipMemcpyAsync(dst, static_cast<const char*>(src) + offset, bytes, hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::copy(const void* src, size_t src_off, void* dst, size_t dst_off, size_t bytes) {
  if (!bytes) return;
  HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + dst_off, static_cast<const char*>(src) + src_off, bytes,
                           hipMemcpyDeviceToDevice, stream_));
}

void Backend::finish() {
  XTG_CHECK(!capturing_, "finish: not during a graph capture");
  HIP_CHECK(hipStreamSynchronize(stream_));
}

std::string Backend::info_json() const {
  hipDeviceProp_t p;
  HIP_CHECK(hipGetDeviceProperties(&p, device_));
  std::string name = p.name;
  for (char& ch : name)
    if (ch == '"' || ch == '\\') ch = ' ';
  return strf("{\"abi\": %d, \"device\": %d, \"name\": \"%s\", \"arch\": \"%s\", \"cus\": %d, \"hbm_bytes\": %zu, "
              "\"weight_bytes\": %zu, \"weights\": %zu}",
              XTG_HIP_ABI_VERSION, device_, name.c_str(), p.gcnArchName, p.multiProcessorCount, size_t(p.totalGlobalMem),
              weight_bytes_, weights_.size());
}

}  // namespace xtg::hip
