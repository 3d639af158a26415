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

#include "attention.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "rows.hpp"
#include "xtg_hip.h"

namespace xtg::hip {

// Rows of one device matmul call (prefill chunks), and of one pass of the host-synchronous call.
constexpr int kMaxDeviceRows = 4096, kHostPassRows = 512;

class Backend {
 public:
  explicit Backend(int device);
  ~Backend();
  Backend(const Backend&) = delete;
  Backend& operator=(const Backend&) = delete;

  // opencl.h:32 prepare(): idempotent, keyed by w.codes
  const PackedNvfp4& prepare(const xtg_nvfp4& w);
  bool has_weight(const uint8_t* codes) const { return weights_.count(codes) != 0; }
  // drops the device copy; refused while a Dory session holds the weight
  void release_weight(const uint8_t* codes);
  // Dory sessions hold the prepared weights they run on (NVFP4 codes or BF16 data as the key). A session that found
  // the weight unprepared owns it: the device copy goes once the last holder lets go and some holder owned it, so
  // a session's teardown never frees weights another session still runs on.
  void hold(const void* key, bool owned);
  void unhold(const void* key);
  // the prepared tiles of the weight keyed by codes, to host memory (bytes = their size)
  void read_tiles(const uint8_t* codes, void* out, size_t bytes);
  // opencl.h:34 host matmul: upload, compute, read back (up to kHostPassRows rows per pass)
  void matmul(const xtg_nvfp4* ws, int nw, const float* x, int m, float* const* ys);
  // opencl.h:54-55 device matmul into consecutive [m][n_i] blocks from y_off
  void matmul_dev(const xtg_nvfp4* ws, int nw, const void* x, int x_dtype, int m, float* y, size_t y_off);
  // the two halves of matmul_dev: the activation operand ([xop][8 row scales], op_bytes(k)) and the GEMV on it
  static size_t op_bytes(int k) { return op_group_bytes(k); }   // per 8 rows
  void prep_x(const void* x, int x_dtype, int m, int k, void* op, float* copy = nullptr);   // copy: FP32 rows too
  // col_scale (device, single weight): y[.][n] *= col_scale[n]. ksplit = 2 (2..8 rows; kernels.hpp GemvCall): the
  // GEMV's K in two halves, the second half's outputs one output set later (m times the weights' total n floats);
  // returns the output sets written (1 or 2: more rows than 8 take the GEMM, whole)
  int matmul_op(const xtg_nvfp4* ws, int nw, const void* op, int m, float* y, size_t y_off,
                const float* col_scale = nullptr, int ksplit = 1);
  // The one-token decode step's projections with its norms riding on them (kernels.hpp FusedGemv; m = 1): the weights,
  // m and the output y (consecutive [m][n_i] blocks; one [m][n] block for a SwiGLU pair) go into f.c; with kInOp,
  // op is the prepared operand. Returns the launch's work-group count: the records a consumer takes.
  int matmul_fused(const xtg_nvfp4* ws, int nw, FusedGemv f, const void* op, int m, float* y);

  // opencl.h:33, 35, 56: the BF16 weight path (keyed by w.data)
  const PackedBf16& prepare(const xtg_bf16& w);
  bool has_bf16(const uint16_t* data) const { return bf16_weights_.count(data) != 0; }
  void release_bf16(const uint16_t* data);
  void matmul_bf16(const xtg_bf16& w, const float* x, int m, float* y);   // host x, y; any m
  // device x [m][k] (x_dtype) into device y + y_off; col_scale (device, optional): y[.][n] *= col_scale[n]
  void matmul_bf16_dev(const xtg_bf16& w, const void* x, int x_dtype, int m, float* y, size_t y_off,
                       const float* col_scale = nullptr);

  // KV caches (xtg::KvCache, kv.h:21-62): device storage, host-side load / save for tests and snapshots
  DevKv* kv_create(int kv_heads, int head_dim, long long slots, int ring, int dtype);
  void kv_destroy(DevKv* c);
  void kv_store(DevKv* c, long long pos, int n, const float* k, const float* v);            // device k, v
  void kv_load(const DevKv* c, int h, long long p0, long long p1, float* k, float* v);      // host k, v
  size_t kv_bytes(const DevKv* c) const;
  void kv_save(const DevKv* c, void* out, size_t bytes);
  void kv_restore(DevKv* c, const void* in, size_t bytes);
  void kv_release(DevKv* c);
  // device copy of src's whole state (data, scales, slot positions) into dst of the same shape and dtype; queued
  void kv_copy(const DevKv* src, DevKv* dst);
  // attention(pool, AttnArgs) (kv.h:64-79) over a device cache; q / k / v / out are device memory
  void attention(const DevKv* c, int n_q, long long pos0, int heads, int window, float scale, const float* q,
                 const float* k, const float* v, float* out);
  // The same with the split partials in the device's fixed scratch (attn_scratch_ptr): allocates nothing (profiling
  // events only while profiling is on); refuses a call whose partials exceed kAttnScratchBytes, and calls while
  // another open backend on the device holds the array (attn_scratch_claim: the first caller keeps it until closed).
  void attention_noalloc(const DevKv* c, int n_q, long long pos0, int heads, int window, float scale, const float* q,
                         const float* k, const float* v, float* out);
  // The attention half of a Dory sublayer (packs/dory/dory.cpp:482-515) on device rows q [m][heads][d],
  // k / v [m][kv_heads][d], g [m][heads * d]: RoPE + norms of q (rewritten) and k, the attention over the cache
  // and this call's keys, the store of k / v into the cache, then out (optional) and op (optional, the
  // o-projection's operand) = justnorm(attention * sigmoid(g * gscale)). Up to 8 rows (a decode or verify step)
  // in one fused producer; more (a prefill chunk): k is rewritten too, and the steps run as separate launches.
  // store = false leaves the cache as it was (a last_loop session's earlier loops, packs/dory/dory.cpp:534-537).
  // gate_rec (one row only): out gets the gated attention before its justnorm and gate_rec [heads] each head's sum
  // of squares, the records of a kInNorm o-projection (kernels.hpp FusedGemv); op must be NULL.
  void attn_step(DevKv* c, int m, long long pos0, int heads, int window, float scale, float theta, float* q,
                 float* k, const float* v, const float* qscale, const float* g, const float* gscale, float* out,
                 void* op, bool store = true, float* gate_rec = nullptr);
  // the row kernels of the decode step (rows.hip); device memory. op (optional): also write the result rows as a
  // GEMV / GEMM operand of ceil(rows / 8) groups of op_bytes(w) bytes.
  void qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0, float theta,
                    const float* qscale);
  // part (floats, optional): the second output set of a K-split matmul_op to add to o (to g and u)
  void slerp_norm(float* x, const float* o, const float* lr, int rows, int w, void* op = nullptr, size_t part = 0);
  void swiglu_norm(const float* g, const float* u, const float* sg, const float* su, int rows, int w, float* out,
                   void* op = nullptr, size_t part = 0);
  void gate_norm(const float* a, const float* gate, const float* gs, int rows, int w, float* out, void* op = nullptr);
  void add_norm(const float* a, const float* b, float* out, int rows, int w, void* op = nullptr);
  // greedy decoding's token (xtg::argmax, sampler.cpp:8-13) of each of `rows` rows of n logits; device out int32
  void argmax(const float* x, int rows, int n, int* out);
  // xtg::Sampler::sample (sampler.cpp:40-94) of each row with the caller's draws u[rows] (host, [0, 1): the
  // generate_canonical the reference's uniform_real_distribution scales by the total); temperature <= 0: argmax
  void sample(const float* x, int rows, int n, float temperature, float top_p, int top_k, float min_p,
              const double* u, int* out);
  // 1 / theta^(2i/d) in FP32 computed on the host as engine/src/kernels.cpp:191-201 does, kept on the device
  const float* inv_freq(float theta, int d);
  // the RoPE rows (cos, sin) of positions 0 .. n - 1 for (theta, d), n >= n_pos (launch_rope_table): made on the
  // device once and grown by doubling when a call needs more positions (not during a graph capture; a table a graph
  // holds is retired until no graph exists). The decode step's producer and scan read their angles from it.
  const float2* rope_table(float theta, int d, long long n_pos);

  // the streaming-read probe (tests/gpu_probe.cpp:59-66's readsum): out (device) gets read_probe_groups(bytes)
  // XOR partials of src's bytes; queued
  void read_probe(const void* src, size_t bytes, uint32_t* out);

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

  // Per-kernel device time (the reference's XTG_GPU_PROFILE, opencl.cpp:293-315): with profiling on (mode 1, or 2
  // to list every launch in queue order as well), every launch is bracketed by two events on the stream; report()
  // waits, sums the durations per kernel name and starts over.
  void set_profile(int mode);
  std::string profile_report();

  // HIP graphs over the backend's stream: begin/end capture every launch queued in between into one graph,
  // launch() replays it. Scratch buffers must already be large enough (run the calls once before capturing).
  // While any graph exists, device memory the backend would free (scratch outgrown by a later call, released
  // weights, buffers and caches) is kept, since a graph may address it, and freed when the last graph goes.
  void graph_begin();
  hipGraphExec_t graph_end(const std::string& name);   // name: the graph's entry in the profile report
  void graph_launch(hipGraphExec_t g);
  void graph_destroy(hipGraphExec_t g);
  bool capturing() const { return capturing_; }
  // Runs fn, which queues one kernel and returns its name, between two profile events when profiling is on.
  template <class F>
  void timed(F&& fn) {
    if (!profile_) {
      fn();
      return;
    }
    hipEvent_t a = event(), b = event();
    HIP_CHECK(hipEventRecord(a, stream_));
    std::string name = fn();
    HIP_CHECK(hipEventRecord(b, stream_));
    pending_.push_back({name, a, b});
  }

 private:
  void ensure(void*& buf, size_t& size, size_t need);
  void check_attention(const DevKv* c, int n_q, long long pos0, const float* q, const float* k, const float* v,
                       const float* out) const;
  // the attention call's launches on partials `part`: for a call of one row block with cached keys to scan, its own
  // keys and the scan in one launch and the merge by heads (XTG_ATTN_UNFUSED=1: the three launches below); else
  // the own keys, the scan and the merge
  void attention_launches(const DevKv* c, const AttnPlan& p, int n_q, long long pos0, int heads, int window,
                          float scale, const float* q, const float* k, const float* v, float* out, float* part);
  void* attn_scratch_ = nullptr;   // this device's fixed attention scratch (device address)
  float2* ident_rope_ = nullptr;   // one RoPE row of 128 identity pairs (cos 1, sin 0): q and k taken as they are
  // frees device memory now (after queued work), or retires it until no graph exists
  void dev_free(void* p);
  void drop_weight(const void* key);
  struct Hold {
    int count = 0;
    bool owned = false;
  };
  std::unordered_map<const void*, Hold> holds_;
  std::vector<void*> retired_;
  void clear_kv(DevKv* c);
  void snapshot(const DevKv* c, void* out);   // kv_bytes(c) host bytes
  hipEvent_t event();
  struct Pending {
    std::string name;
    hipEvent_t a, b;
  };
  int profile_ = 0;
  bool capturing_ = false;
  std::unordered_map<hipGraphExec_t, std::string> graphs_;
  std::vector<Pending> pending_;
  std::vector<hipEvent_t> free_events_;
  struct Total {
    long calls = 0;
    double ms = 0;
  };
  std::vector<std::pair<std::string, Total>> totals_;
  int device_ = 0;
  hipStream_t stream_ = nullptr;
  std::unordered_map<const uint8_t*, PackedNvfp4> weights_;
  std::unordered_map<const uint16_t*, PackedBf16> bf16_weights_;
  void* opb_ = nullptr;    // the BF16 GEMV's activation operand
  size_t opb_size_ = 0;
  std::unordered_set<void*> allocs_;
  size_t weight_bytes_ = 0;
  // scratch (grown on demand, owned): activation operand, its row scales, host-call staging
  void* op_ = nullptr;
  size_t op_size_ = 0;
  void* part_ = nullptr;   // attention split partials
  size_t part_size_ = 0;
  void* kproc_ = nullptr;  // processed k rows of a decode step whose store follows the scan
  size_t kproc_size_ = 0;
  void* sample_ = nullptr;   // sampling scratch: weights and the radix sort's buffers
  size_t sample_size_ = 0;
  std::unordered_set<DevKv*> kvs_;
  std::vector<std::pair<std::pair<float, int>, float*>> inv_freq_;
  struct RopeTable {
    float theta;
    int d;
    long long n;
    float2* p;
  };
  std::vector<RopeTable> rope_;
  void* hx_ = nullptr;
  size_t hx_size_ = 0;
  void* stage_ = nullptr;   // a weight's checkpoint arrays on their way to the tile layout
  size_t stage_size_ = 0;
  static constexpr size_t kStageBytes = size_t(64) << 20;
  void* hy_ = nullptr;
  size_t hy_size_ = 0;
};

}  // namespace xtg::hip
