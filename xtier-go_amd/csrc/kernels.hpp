// Host-side launchers of the gfx950 kernels (the kernels themselves live in the .hip files).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace xtg::hip {

// ---- NVFP4 GEMV / skinny GEMM (gemv.hip) ----
//
// Device weight layout: tiles of 16 rows x 128 inputs, 1152 bytes each, row-block major ([rb][kt]):
//   bytes    0..1023: lane l's 16 bytes at 16 l = the codes of row rb*16 + (l & 15), inputs
//                     kt*128 + 32 (l >> 4) .. +32 (the original bytes, low nibble = even input)
//   bytes 1024..1151: lane l's 2 bytes at 1024 + 2 l = that row's two E4M3 scales for those 32 inputs
// Rows past n_out and inputs past k are zero codes with zero scales.
constexpr int kTileRows = 16, kTileK = 128, kTileBytes = 1152;

struct PackedNvfp4 {
  uint8_t* tiles = nullptr;   // device
  size_t bytes = 0;
  int n = 0, k = 0, nb = 0, kt = 0;
  float global = 1.f;
};

// Device repack of [n][k/2] codes and [n][k/16] scales (device copies of the checkpoint's arrays, 8-byte aligned)
// into the tile layout above.
std::string launch_pack_nvfp4(const uint8_t* codes, const uint8_t* scales, int n, int k, uint8_t* tiles,
                              hipStream_t stream);

// The MFMA operand form of the activations: [kt][4 steps][64 entries][8 f16] (4096 bytes per k-tile). Operand
// column 2 r is the high f16 part of row r scaled by 2^s_r, column 2 r + 1 the low part; xinv[r] = 2^-s_r. Entry
// 4 c + g of step t holds column c's inputs 32 g + 8 t .. +8 of the k-tile, so the live columns of m rows fill the
// first 128 m bytes of every step (one cache line per step at m = 1).
inline size_t xop_bytes(int k) { return size_t((k + kTileK - 1) / kTileK) * 4096; }
constexpr int kMaxRows = 8;
constexpr int kMaxOperandRows = 4096;   // rows of one grouped operand (the GEMM's limit)
// One group's operand: xop_bytes(k), then its 8 row factors xinv. m rows take ceil(m / 8) consecutive groups.
inline size_t op_group_bytes(int k) { return xop_bytes(k) + kMaxRows * sizeof(float); }

enum XDtype { kXF32 = 0, kXBF16 = 1 };
// Launchers return the kernel's name (as rocprof prints it, without the namespace) for the profiler.
// The operand of m >= 1 rows into op (ceil(m / 8) groups of op_group_bytes(k)).
std::string launch_prep_x(const void* x, int x_dtype, int m, int k, void* op, hipStream_t stream,
                          float* copy = nullptr);

struct GemvCall {
  const PackedNvfp4* w[4] = {nullptr, nullptr, nullptr, nullptr};
  int nw = 0;
  size_t y_off[4] = {0, 0, 0, 0};   // floats from y
  const float* col_scale[4] = {nullptr, nullptr, nullptr, nullptr};   // optional per-column factors (device)
  float* y = nullptr;
  int m = 0;
  const void* xop = nullptr;
  const float* xinv = nullptr;
  const void* x = nullptr;   // raw rows [m][k] (x_dtype) in place of a prepared operand: the GEMV builds its own
  int x_dtype = 0;
  int k = 0;
  int parts = 2;   // the GEMM's activation parts (prefill chunks): 2, high and low f16; 1, the high part alone
  // the GEMV on a prepared operand (2..8 rows): 2 splits K in two halves whose partial outputs go to y (the first
  // k-tiles) and to y + y_part (the rest), each laid out as y_off says; the consumer adds them, first + second.
  // Each work-group then reads half of the rows' operand (the bytes its k-range needs), the share of a launch that
  // grows with the rows. 1: one output set.
  int ksplit = 1;
  size_t y_part = 0;
};
// The launch shape: R row-blocks and T k-tiles per wave, S waves per work-group along k.
struct GemvShape {
  int r = 1, t = 1, s = 1;
};
GemvShape gemv_shape(int kt, const int* nbs, int nw, int m, bool raw = false);   // raw: BF16 rows read as they are
std::string launch_gemv(const GemvCall& c, hipStream_t stream);
// whether launch_gemv takes c's raw rows for its shape (otherwise prepare the operand first)
bool gemv_takes_raw(const GemvCall& c);

// ---- the one-token decode step's projections with the nGPT norms riding on them (gemv.hip) ----
//
// A norm over a whole row needs every output of the projection that made the row, so as a kernel of its own it
// costs a dependent launch per norm. Here the producing GEMV writes, besides its outputs, one record of partial
// sums per work-group over the outputs it owns (records [Q quantities][groups]), and the consuming GEMV adds the
// P records in a fixed order (every work-group the same order: bit-identical factors). One activation row (m = 1).
//   input side:  kInOp     the prepared operand (c.xop / c.xinv)
//                kInSlerp  W x_new with x_new = (ya + lr (yb - ya)) f2, ya = x fa, yb = o fb (kernels.cpp:177-189),
//                          taken in its linear form f2 (fa W a + fb W b), a = (1 - lr) x, b = lr o: the producer
//                          writes a and b as an operand (c.xop: high and low f16 parts of a 2^ea in columns 0, 1 and
//                          of b 2^eb in 2, 3; in_ia = 2^-ea, in_ib = 2^-eb), so the math waits for no factor; the
//                          factors come from kOutSlerp records in the epilogue: fa = 1/sqrt(sum x^2 + 1e-6), fb
//                          likewise of o, f2 of sum t^2 = fa^2 sum (1-lr)^2 x^2 + 2 fa fb sum (1-lr) lr x o + fb^2
//                          sum lr^2 o^2; each work-group also writes its share of x_new to in_xout (the next residual)
//                          from in_x, in_o, in_lr. in_post folds one more row norm of x_new into f2 (sum x_new^2 =
//                          f2^2 sum t^2): kPostAddNorm x_new := justnorm(x_new + x_new) (a loop's entry with state
//                          = input), kPostNorm x_new := justnorm(x_new) (a loop's exit)
//                kInNorm   h r, r = 1/sqrt(sum h^2 + 1e-6) from kOutSwiglu records, built from the row h (in_x) lane
//                          by lane (unit norm: a fixed operand exponent 2^14, |h r| <= 1)
//   output side: kOutPlain
//                kOutSlerp  y as usual, plus records of sum x^2, o^2, (1-lr)^2 x^2, (1-lr) lr x o, lr^2 o^2 over the
//                           group's outputs o (out_x: the residual [n], out_lr [n]); one weight; with out_op, the
//                           kInSlerp operand of a = (1 - lr) x and b = lr o at out_ea = 2^ea, out_eb = 2^eb (exponents
//                           that keep |a 2^ea|, |b 2^eb| <= 2^14; the buffer's entries for inputs past n stay zero)
//                kOutSwiglu two weights (gate, up) of equal shape, the same row-blocks of both in one work-group:
//                           y = h = silu(g sg) (u su) [n] (kernels.cpp:225-234) and records of sum h^2
enum { kInOp = 0, kInSlerp = 1, kInNorm = 2 };
enum { kOutPlain = 0, kOutSlerp = 1, kOutSwiglu = 2 };
enum { kPostNone = 0, kPostAddNorm = 1, kPostNorm = 2 };
struct FusedGemv {
  GemvCall c;                        // weights, y, m = 1, k (kInOp: c.xop / c.xinv)
  int in = kInOp, out = kOutPlain;
  const float* in_x = nullptr;       // kInSlerp: x [k]; kInNorm: h [k]
  const float* in_o = nullptr;       // kInSlerp: o [k]
  const float* in_lr = nullptr;      // kInSlerp: lr [k]
  const float* in_part = nullptr;    // the producing launch's records
  int in_groups = 0;                 // their number (fused_gemv_groups of that launch)
  float* in_xout = nullptr;          // kInSlerp: where x_new goes
  float in_ia = 1.f, in_ib = 1.f;    // kInSlerp: 2^-ea, 2^-eb
  int in_post = 0;                   // kInSlerp: kPostNone, kPostAddNorm or kPostNorm
  const float* out_x = nullptr;      // kOutSlerp
  const float* out_lr = nullptr;
  const float* out_sg = nullptr;     // kOutSwiglu
  const float* out_su = nullptr;
  float* out_part = nullptr;         // kOutSlerp / kOutSwiglu: the records (5 or 1 x kMaxFusedGroups floats)
  void* out_op = nullptr;            // kOutSlerp: the consumer's kInSlerp operand (xop_bytes(n) bytes), or NULL
  float out_ea = 1.f, out_eb = 1.f;  // its factors 2^ea, 2^eb
};
int fused_gemv_groups(const FusedGemv& f);
// Why launch_gemv_fused cannot take f's weights, rows, kinds and record count (no kernel made for the launch shape,
// more waves or records than a launch holds), or "" when it can; pointers are not looked at.
std::string fused_gemv_unsupported(const FusedGemv& f);
constexpr int kMaxFusedGroups = 1024;   // work-groups of a launch whose records a consumer takes
std::string launch_gemv_fused(const FusedGemv& f, hipStream_t stream);

// ---- NVFP4 GEMM for prefill chunks of m > 8 rows (gemm.hip) ----
// The same weights and call description (c.xop: group 0 of ceil(m / 8) operand groups of op_group_bytes(k);
// c.xinv unused), any m >= 1; y[i] blocks as in the GEMV.
std::string launch_gemm(const GemvCall& c, hipStream_t stream);

// ---- BF16 GEMV / skinny GEMM (gemv_bf16.hip) ----
//
// Device weight layout: tiles of 16 rows x 128 inputs, 4096 bytes each, row-block major ([rb][kt]): step s
// (inputs 32 s .. 32 s + 31 of the tile) at 1024 s, lane l's 8 BF16 at 1024 s + 16 l = row rb*16 + (l & 15),
// inputs kt*128 + 32 s + 8 (l >> 4) .. +8. Rows past n_out and inputs past k are zeros.
constexpr int kBf16TileBytes = 4096;

struct PackedBf16 {
  uint16_t* tiles = nullptr;   // device
  size_t bytes = 0;
  int n = 0, k = 0, nb = 0, kt = 0;
};

void pack_bf16_tiles(const uint16_t* w, int n, int k, std::vector<uint16_t>& out);
// The activations as MFMA B operands: [kt][4 steps][2 column blocks][64 entries][8 BF16]; column 3 r + t of block
// cb is term t of row 5 cb + r (the three BF16 terms sum to the FP32 row), entry 4 column + g holds inputs
// 32 step + 8 g .. +8 of the k-tile.
inline size_t xop_bf16_bytes(int k) { return size_t((k + kTileK - 1) / kTileK) * 8192; }
std::string launch_prep_x_bf16(const void* x, int x_dtype, int m, int k, void* xop, hipStream_t stream);
GemvShape gemv_bf16_shape(int kt, int nb, int m);
// y [m][n] (+ optional per-column factors col_scale[n]) from the operand of m <= 8 rows.
std::string launch_gemv_bf16(const PackedBf16& w, const void* xop, int m, float* y, const float* col_scale,
                             hipStream_t stream);

// ---- the streaming-read probe (probe.hip) ----
// XOR fold of bytes (a multiple of 16) of device memory in 16-byte loads: one uint32 partial per work-group into out
// (read_probe_groups(bytes) of them).
size_t read_probe_groups(size_t bytes);
std::string launch_read_probe(const void* src, size_t bytes, uint32_t* out, hipStream_t stream);

// ---- sampling (sample.hip) ----
constexpr int kMaxSampleRows = 8;
// xtg::Sampler::sample for rows of device logits [rows][n] with the caller's uniform draws u[rows] (host, [0, 1)),
// temperature > 0; device tokens out[rows]. scratch: sample_scratch_bytes(rows, n) device bytes.
size_t sample_scratch_bytes(int rows, int n);
std::string launch_sample(const float* logits, int rows, int n, float temperature, float top_p, int top_k,
                          float min_p, const double* u, int* out, void* scratch, hipStream_t stream);
// xtg::argmax over slices of the rows (rows <= kMaxSampleRows; scratch: sample_scratch_bytes(rows, n))
std::string launch_argmax_slices(const float* logits, int rows, int n, int* out, void* scratch, hipStream_t stream);

}  // namespace xtg::hip
