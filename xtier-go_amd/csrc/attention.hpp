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
  uint16_t* k = nullptr;    // kv_heads * slots_pad * head_dim BF16
  uint16_t* v = nullptr;
  int* slot_pos = nullptr;  // slots_pad, -1 = empty
};

// Element offsets of (head, slot, dim) in the K and V layouts (for host-side load / save).
size_t kv_k_index(int h, int slot, int dim, int slots_pad, int d);
size_t kv_v_index(int h, int slot, int dim, int slots_pad, int d);

// The rows of positions pos .. pos + n - 1 from FP32 device k, v [n][kv_heads][head_dim]; a ring keeps the last
// `slots` rows.
void launch_kv_store(const DevKv& c, long long pos, int n, const float* k, const float* v, hipStream_t stream);

struct AttnPlan {
  int group = 1, qb = 1;         // q heads per KV head; 16-column blocks of (row, head) pairs
  int tile_lo = 0, tiles = 0;    // the 32-slot tiles to scan
  int splits = 1;                // work-groups per KV head
};
AttnPlan attn_plan(const DevKv& c, int n_rows, int heads, long long pos0, int window);
size_t attn_part_floats(int kv_heads, int splits, int qcols_pad, int d);
// Query rows per launch (at most 32 (row, head) columns per KV head) and the partial buffer a call needs.
int attn_rows_per_block(int group);
size_t attn_part_floats_max(const DevKv& c, int n_q, int heads, long long pos0, int window);
// One block of n_rows <= attn_rows_per_block query rows (rows row0 .. row0 + n_rows - 1 of a call with n_own new
// rows; device q / k / v as xtg::AttnArgs, engine/include/xtg/kv.h:67-78): the split partials into part, then
// their merge into out (the block's rows). Launchers return the kernel name.
std::string launch_attn_decode(const DevKv& c, const AttnPlan& p, const float* q, const float* k, const float* v,
                               int n_rows, int row0, int n_own, int heads, long long pos0, int window, float scale,
                               float* part, hipStream_t stream);
std::string launch_attn_merge(const DevKv& c, const AttnPlan& p, int n_rows, int heads, const float* part, float* out,
                              hipStream_t stream);

}  // namespace xtg::hip
