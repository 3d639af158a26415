// Device KV cache and decode attention launchers (attention.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace xtg::hip {

// One KV cache instance (xtg::KvCache, engine/include/xtg/kv.h:21-62) in device memory. slots: the capacity (the
// ring size for a ring); slots_pad: slots rounded up to 32. Layouts are described in attention.hip.
struct DevKv {
  int kv_heads = 0, head_dim = 0;
  long long slots = 0;
  int slots_pad = 0;
  bool ring = false;
  bool fp8 = false;            // E4M3 codes + an FP32 scale per (slot, head) (kv.cpp:94-108), else BF16
  void* k = nullptr;           // kv_heads * slots_pad * head_dim elements (2 bytes BF16, 1 byte FP8)
  void* v = nullptr;
  float* kscale = nullptr;     // FP8: [kv_heads][slots_pad]
  float* vscale = nullptr;
  int* slot_pos = nullptr;     // slots_pad, -1 = empty
  size_t elems() const { return size_t(kv_heads) * size_t(slots_pad) * size_t(head_dim); }
  size_t data_bytes() const { return elems() * (fp8 ? 1 : 2); }
  size_t scale_bytes() const { return fp8 ? size_t(kv_heads) * size_t(slots_pad) * sizeof(float) : 0; }
};

// Element offsets of (head, slot, dim) in the K and V layouts (for host-side load / save), BF16 and FP8.
size_t kv_k_index(int h, int slot, int dim, int slots_pad, int d);
size_t kv_v_index(int h, int slot, int dim, int slots_pad, int d);
size_t kv_k8_index(int h, int slot, int dim, int slots_pad, int d);
size_t kv_v8_index(int h, int slot, int dim, int slots_pad, int d);

// The rows of positions pos .. pos + n - 1 from FP32 device k, v [n][kv_heads][head_dim]; a ring keeps the last
// `slots` rows.
std::string launch_kv_store(const DevKv& c, long long pos, int n, const float* k, const float* v,
                            hipStream_t stream);

// How one attention call (n_q query rows at pos0) is cut up. Query rows go in blocks of rpb rows (at most 32
// (row, head) columns per KV head); each block's key tiles go to `splits` work-groups per KV head, plus `own`
// partials per (block, KV head) for this call's own keys (one per chunk of kOwnChunk keys of a column tile's key
// range; chunks with no key leave an empty record, sum 0). Partials: acc [blocks][kv_heads][splits + own][qpad][d]
// then (max, sum) [blocks][kv_heads][splits + own][qpad][2]; q-col (row r of the block, head g of the group) is
// r * group + g.
constexpr int kOwnChunk = 128;
struct AttnPlan {
  int group = 1;               // q heads per KV head
  int rpb = 1, blocks = 1;     // rows per block, blocks
  int qpad = 16;               // q-cols per block, padded to 16
  int tile_lo = 0, tiles = 0;  // the 32-slot tiles to scan
  int splits = 0;              // work-groups per KV head over the tiles (0: no cached key is visible)
  int own = 1;                 // own-key records per (block, KV head, q-col), after the splits'
  int kv_heads = 1, d = 64;
  size_t records() const { return size_t(blocks) * size_t(kv_heads) * size_t(splits + own) * size_t(qpad); }
  size_t part_floats() const { return records() * size_t(d + 2); }
};
AttnPlan attn_plan(const DevKv& c, int n_q, int heads, long long pos0, int window);

// For blocks b0 .. b0 + nblocks - 1 (block b: rows b * rpb .. of the call; device q / k / v as xtg::AttnArgs,
// engine/include/xtg/kv.h:67-78), one launch each: the own-key partials and the split partials. Then the merge of
// every row into out [n_q][heads][d].
std::string launch_attn_own(const AttnPlan& p, int b0, int nblocks, const float* q, const float* k, const float* v,
                            int n_q, int heads, int window, float scale, float* part, hipStream_t stream);
std::string launch_attn_scan(const DevKv& c, const AttnPlan& p, int b0, int nblocks, const float* q, int n_q,
                             int heads, long long pos0, int window, float scale, float* part, hipStream_t stream);
std::string launch_attn_merge(const AttnPlan& p, int n_q, int heads, const float* part, float* out,
                              hipStream_t stream);

// The split partials of the attention call that allocates nothing live in a fixed device array of this many bytes
// per device (attention.hip), loaded with the code object and held until the process ends. attn_scratch_ptr(device)
// is its device address on `device`, which must be the current device; the first call per device looks it up.
constexpr size_t kAttnScratchBytes = size_t(16) << 20;
void* attn_scratch_ptr(int device);
// The array of a device belongs to one backend at a time: the first that claims it keeps it until it lets go (at
// its close), and a claim from another backend on that device is refused (false), since their calls would race on
// the one array. Claiming again from the holder succeeds.
bool attn_scratch_claim(int device, const void* owner);
void attn_scratch_let_go(int device, const void* owner);

constexpr int kProdRows = 8, kProdGroup = 8;   // the producer's rows per call and q heads per KV head

// The RoPE rows of positions 0 .. n_pos - 1 into out [n_pos][d / 2]: (cos, sin) of FP32(pos) * inv_freq[i]
// (engine/src/kernels.cpp:203-222). The producer and the decode step's scan read their rows' angles from it.
std::string launch_rope_table(const float* inv_freq, int d, long long n_pos, float2* out, hipStream_t stream);
// The decode step's producer (packs/dory/dory.cpp:482-490 and the cache store of :507): in one launch per
// call (m <= 8 rows), RoPE (angles from the table rope, covering positions pos0 .. pos0 + m - 1) + justnorm of
// q and k (q *= qscale, q written back in place; k read only, the processed rows also written to kout when it is
// not NULL), the own-key partials from the FP32 rows, and -- when store is set -- k, v stored into the cache. Storing before the scan is exact when no key the scan should see is
// overwritten: a linear cache, or a ring of at least window + m - 1 slots.
std::string launch_qk_produce(const DevKv& c, const AttnPlan& p, float* q, const float* k, const float* v, float* kout,
                              int m, int heads, long long pos0, int window, float scale, const float2* rope,
                              const float* qscale, bool store, float* part, hipStream_t stream);
// The producer and the scan in one launch (same arguments and results as launch_qk_produce followed by
// launch_attn_scan, except that q is not written back): for a call of one row block with cached keys to scan
// (attn_step_fuses). The store may run concurrently with the scan only under the store-first condition above;
// otherwise pass store = false and kout, and store after.
// plain: q and k as they are (no RoPE, norms, qscale, store or kout; rope one identity row, cos 1 and sin 0): the
// attention call's own keys and scan in one launch, for a call that attn_step_fuses.
bool attn_step_fuses(const AttnPlan& p, int m);
std::string launch_attn_step(const DevKv& c, const AttnPlan& p, float* q, const float* k, const float* v,
                             float* kout, int m, int heads, long long pos0, int window, float scale,
                             const float2* rope, const float* qscale, bool store, float* part,
                             hipStream_t stream, bool plain = false);
// The decode step's finish (dory.cpp:509-515): every row's merge, times sigmoid(g * gscale), justnorm over the
// heads, written to out (optional) and as a GEMV operand (optional, Backend::op_bytes(heads * d) bytes).
std::string launch_attn_gate(const AttnPlan& p, int m, int heads, const float* part, const float* g, const float* gs,
                             float* out, void* op, hipStream_t stream);
// The same for one row with the justnorm left to the consumer: y [heads * d] = the gated merge before its norm, and
// rec [heads] = each head's sum of squares (the records a kInNorm projection takes, kernels.hpp FusedGemv).
std::string launch_attn_gate_heads(const AttnPlan& p, int heads, const float* part, const float* g, const float* gs,
                                   float* y, float* rec, hipStream_t stream);
// The attention call's merge (launch_attn_merge) for a call of one row block, by heads: one work-group per (head,
// row) merges that head's records with one to four waves, out [n_q][heads][d] (16-byte aligned).
std::string launch_attn_merge_heads(const AttnPlan& p, int n_q, int heads, const float* part, float* out,
                                    hipStream_t stream);

}  // namespace xtg::hip
