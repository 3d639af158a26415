// The looped-nGPT (Dory) decode step on the HIP backend: the composition of packs/dory/dory.cpp:467-578
// (DorySession::sublayer / run_chunk / forward; the OpenCL GpuDorySession, dory.cpp:1108-1214) over the gfx950
// kernels. Weights are prepared once; every forward call queues its kernels on the backend's stream, so a step
// can be captured into one HIP graph.
#pragma once

#include <string>
#include <vector>

#include "backend.hpp"
#include "xtg_hip.h"

namespace xtg::hip {

class DorySession {
 public:
  DorySession(Backend& b, const xtg_dory_config& c, const xtg_dory_layer* layers, const xtg_nvfp4& head,
              const float* logit_scale);
  ~DorySession();
  DorySession(const DorySession&) = delete;
  DorySession& operator=(const DorySession&) = delete;

  // run_chunk from the hidden rows x [m][hidden] (device; the embedding rows) at positions pos0 .. pos0 + m - 1,
  // then the LM head times logit_scale into logits [m][vocab] (device). m <= 512. The caches gain the chunk's keys.
  void forward(const float* x, int m, long long pos0, float* logits);
  // DorySession::forward (dory.cpp:554-578) over n rows in chunks of up to 512, with logits for all rows
  // ([n][vocab]), the last ([vocab]) or none (want: XTG_LOGITS_*).
  void prefill(const float* x, int n, long long pos0, int want, float* logits);
  // A BF16 LM head [vocab][hidden] in place of the NVFP4 one (a BF16 checkpoint's lm_head.weight, dory.cpp:325;
  // the resident GPU session's head matmul, dory.cpp:1203). Not during a graph capture.
  void set_head_bf16(const xtg_bf16& head);
  DevKv* cache(int attn, int inst);
  // DorySession / GpuDorySession::snapshot and restore (dory.cpp:591-614, 1231-1273): device copies of every ring
  // cache into snapshot slot `slot` (storage made on its first use) and back. Global caches need no copy: what a
  // later call wrote past the restored position is masked by position. The caller keeps the position.
  void snapshot(int slot);
  void restore(int slot);
  Backend& backend() { return b_; }
  int n_attn() const { return n_attn_; }

 private:
  struct Layer {
    xtg_dory_layer w;   // weight descriptors (host pointers key the prepared device copies)
    int attn = -1;
    bool recurrent = false;
    float* qscale = nullptr;   // device copies of the per-layer vectors
    float* gscale = nullptr;
    float* sg = nullptr;
    float* su = nullptr;
    float* lr = nullptr;
    float lin_a = 1.f, lin_b = 1.f;   // 2^ea, 2^eb of the slerp's linear-form operand (kernels.hpp kInSlerp)
  };
  void sublayer(Layer& L, int m, long long pos0, int inst, bool store);
  // the same for a decode or verify step (m <= 8) with the slerp and SwiGLU norms riding on the projections: after
  // it the residual awaits its slerp (pend_), which the next sublayer's first projection (or materialize) makes
  void sublayer_decode(Layer& L, int m, long long pos0, int inst, bool store);
  // the awaited slerp as a launch of its own: x_ and op_h_ hold the residual's rows afterwards
  void materialize(int m);
  // keep_pending: a one-row chunk's last slerp is left for the head's projection (head() makes it)
  void run_chunk(const float* x, int m, long long pos0, bool keep_pending = false);
  void head(int r0, int rows, float* logits);
  float* upload(const float* v, size_t n);
  void build(const xtg_dory_layer* layers, const float* logit_scale);
  void prepare(const xtg_nvfp4& w);
  // why some projection of a one-token step has no fused launch for this model's shapes ("" when all have one): such
  // a model's one-token steps take the separate norm launches
  std::string fused_unsupported();
  void release_all();

  Backend& b_;
  xtg_dory_config c_;
  std::vector<Layer> layers_;
  xtg_nvfp4 head_;            // codes NULL: no NVFP4 head (a BF16 head must be set)
  xtg_bf16 head_bf16_{};      // data non-NULL: the head in use
  float* logit_scale_ = nullptr;
  int n_attn_ = 0;
  std::vector<DevKv*> caches_;   // [attn][loops]
  std::vector<std::vector<DevKv*>> snaps_;   // [slot][ring caches in caches_ order]
  std::vector<void*> owned_;     // device vectors and scratch
  // the weights this session holds on the backend, once per use (a weight it found unprepared goes with the last
  // session holding it: the host arrays that key it may be freed and their addresses reused once it is gone)
  std::vector<const void*> held_;
  // scratch for up to 512 rows (one chunk); x_ / x2_ trade places when a projection writes the next residual
  float *x_ = nullptr, *x2_ = nullptr, *input_ = nullptr, *state_ = nullptr, *proj_ = nullptr, *gu_ = nullptr,
        *o_ = nullptr;
  // the fused one-token path: records of the slerp's and the SwiGLU's partial sums (kernels.hpp FusedGemv), and
  // the residual awaiting its slerp (of o_ with pend_lr_, pend_groups_ records in part_s_)
  float *part_s_ = nullptr, *part_h_ = nullptr;
  float *part_a_ = nullptr, *att_ = nullptr;   // the attention gate's per-head records and gated heads
  bool fused_ = true, pend_ = false;
  bool ksplit_ = true;   // steps of 2..8 rows split K in two in gate/up, down and o (GemvCall::ksplit)
  const float* pend_lr_ = nullptr;
  float pend_a_ = 1.f, pend_b_ = 1.f;   // its linear-form operand's factors, the operand in op_lin_
  int pend_groups_ = 0;
  int pend_post_ = 0;   // a loop boundary's norm of the slerped residual, folded into the consumer (kPost*)
  // GEMV operands, each written by the kernel that produces its rows: x's (K = hidden; by the slerp / loop norms
  // or, for the first sublayer, prep_x), the gated attention's (K = heads * head_dim), the SwiGLU's (K = ffn)
  void* op_h_ = nullptr;
  void* op_q_ = nullptr;
  void* op_f_ = nullptr;
  void* op_last_ = nullptr;   // one row's operand (K = hidden), for the head of a chunk's last row
  void* op_lin_ = nullptr;    // the fused one-token path's slerp operand (K = hidden; kernels.hpp kInSlerp)
};

}  // namespace xtg::hip
