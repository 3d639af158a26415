// HipBackend: the MI355X counterpart of xtg::OpenClBackend (engine/include/xtg/opencl.h:22-63). One device,
// one in-order stream, the device copies of the prepared weights, and the device-resident buffer calls.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "kernels.hpp"
#include "xtg_hip.h"

namespace xtg::hip {

class Backend {
 public:
  explicit Backend(int device);
  ~Backend();
  Backend(const Backend&) = delete;
  Backend& operator=(const Backend&) = delete;

  // opencl.h:32 prepare(): idempotent, keyed by w.codes
  const PackedNvfp4& prepare(const xtg_nvfp4& w);
  void release_weight(const uint8_t* codes);
  // opencl.h:34 host matmul: upload, compute, read back (8 rows per pass)
  void matmul(const xtg_nvfp4* ws, int nw, const float* x, int m, float* const* ys);
  // opencl.h:54-55 device matmul into consecutive [m][n_i] blocks from y_off
  void matmul_dev(const xtg_nvfp4* ws, int nw, const void* x, int x_dtype, int m, float* y, size_t y_off);

  // opencl.h:40-45
  void* alloc(size_t bytes);
  void release(void* p);
  void write(void* dst, size_t offset, const void* src, size_t bytes);
  void read(const void* src, size_t offset, void* dst, size_t bytes);
  void copy(const void* src, size_t src_off, void* dst, size_t dst_off, size_t bytes);
  void finish();

  hipStream_t stream() const { return stream_; }
  int device() const { return device_; }
  std::string info_json() const;
  size_t weight_bytes() const { return weight_bytes_; }

 private:
  void ensure(void*& buf, size_t& size, size_t need);
  int device_ = 0;
  hipStream_t stream_ = nullptr;
  std::unordered_map<const uint8_t*, PackedNvfp4> weights_;
  std::unordered_set<void*> allocs_;
  size_t weight_bytes_ = 0;
  // scratch (grown on demand, owned): activation operand, its row scales, host-call staging
  void* xop_ = nullptr;
  size_t xop_size_ = 0;
  void* xinv_ = nullptr;
  size_t xinv_size_ = 0;
  void* hx_ = nullptr;
  size_t hx_size_ = 0;
  void* hy_ = nullptr;
  size_t hy_size_ = 0;
};

}  // namespace xtg::hip
