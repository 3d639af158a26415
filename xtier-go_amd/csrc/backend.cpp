#include "backend.hpp"

#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace xtg::hip {

Backend::Backend(int device) : device_(device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  XTG_CHECK(device >= 0 && device < count, "no HIP device %d (%d present)", device, count);
  HIP_CHECK(hipSetDevice(device));
  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
}

Backend::~Backend() {
  // teardown: errors cannot be reported from a destructor; every release is still attempted
  (void)hipSetDevice(device_);
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& kv : weights_) (void)hipFree(kv.second.tiles);
  for (void* p : allocs_) (void)hipFree(p);
  for (void* p : {xop_, xinv_, hx_, hy_})
    if (p) (void)hipFree(p);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void Backend::ensure(void*& buf, size_t& size, size_t need) {
  if (size >= need) return;
  if (buf) {
    HIP_CHECK(hipStreamSynchronize(stream_));   // queued work may still read the old buffer
    HIP_CHECK(hipFree(buf));
    buf = nullptr;
    size = 0;
  }
  HIP_CHECK(hipMalloc(&buf, need));
  size = need;
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
  std::vector<uint8_t> host;
  pack_nvfp4_tiles(w.codes, w.scales, w.n_out, w.k, host);
  PackedNvfp4 p;
  p.n = w.n_out;
  p.k = w.k;
  p.nb = (w.n_out + kTileRows - 1) / kTileRows;
  p.kt = (w.k + kTileK - 1) / kTileK;
  p.global = w.global;
  p.bytes = host.size();
  HIP_CHECK(hipMalloc(&p.tiles, p.bytes));
  HIP_CHECK(hipMemcpy(p.tiles, host.data(), p.bytes, hipMemcpyHostToDevice));
  weight_bytes_ += p.bytes;
  return weights_.emplace(w.codes, p).first->second;
}

void Backend::release_weight(const uint8_t* codes) {
  auto it = weights_.find(codes);
  if (it == weights_.end()) return;
  HIP_CHECK(hipStreamSynchronize(stream_));   // queued launches may still read it
  HIP_CHECK(hipFree(it->second.tiles));
  weight_bytes_ -= it->second.bytes;
  weights_.erase(it);
}

void Backend::matmul_dev(const xtg_nvfp4* ws, int nw, const void* x, int x_dtype, int m, float* y, size_t y_off) {
  XTG_CHECK(nw >= 1 && nw <= 4, "matmul: %d weights (1..4 per call)", nw);
  XTG_CHECK(m >= 1 && m <= kMaxRows, "matmul: %d rows (1..%d per device call)", m, kMaxRows);
  XTG_CHECK(x_dtype == kXF32 || x_dtype == kXBF16, "matmul: unknown activation type %d", x_dtype);
  XTG_CHECK(x && y, "matmul: NULL input or output");
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
  ensure(xop_, xop_size_, xop_bytes(k));
  ensure(xinv_, xinv_size_, kMaxRows * sizeof(float));
  launch_prep_x(x, x_dtype, m, k, xop_, static_cast<float*>(xinv_), stream_);
  c.y = y;
  c.m = m;
  c.xop = xop_;
  c.xinv = static_cast<const float*>(xinv_);
  launch_gemv(c, stream_);
}

void Backend::matmul(const xtg_nvfp4* ws, int nw, const float* x, int m, float* const* ys) {
  XTG_CHECK(nw >= 1 && m >= 1 && x, "matmul: %d weights, %d rows", nw, m);
  const int k = ws[0].k;
  for (int i = 0; i < nw; ++i) XTG_CHECK(ws[i].k == k && k % 16 == 0, "matmul: input widths differ (%d, %d)", ws[i].k, k);
  // more than four weights: groups of four, each group one fused launch
  size_t out_per_row = 0;
  for (int i = 0; i < nw; ++i) out_per_row += size_t(ws[i].n_out);
  ensure(hx_, hx_size_, size_t(kMaxRows) * size_t(k) * sizeof(float));
  ensure(hy_, hy_size_, size_t(kMaxRows) * out_per_row * sizeof(float));
  for (int r0 = 0; r0 < m; r0 += kMaxRows) {
    const int rows = std::min(kMaxRows, m - r0);
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
  auto it = allocs_.find(p);
  XTG_CHECK(it != allocs_.end(), "release: %p was not allocated by this backend", p);
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipFree(p));
  allocs_.erase(it);
}

void Backend::write(void* dst, size_t offset, const void* src, size_t bytes) {
  if (!bytes) return;
  HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + offset, src, bytes, hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::read(const void* src, size_t offset, void* dst, size_t bytes) {
  if (bytes)
    HIP_CHECK(hipMemcpyAsync(dst, static_cast<const char*>(src) + offset, bytes, hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

void Backend::copy(const void* src, size_t src_off, void* dst, size_t dst_off, size_t bytes) {
  if (!bytes) return;
  HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + dst_off, static_cast<const char*>(src) + src_off, bytes,
                           hipMemcpyDeviceToDevice, stream_));
}

void Backend::finish() { HIP_CHECK(hipStreamSynchronize(stream_)); }

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
