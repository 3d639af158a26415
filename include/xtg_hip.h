/* xtg_hip: the MI355X (gfx950) kernel layer of the xtier-go decode path, behind a C ABI.
 *
 * One handle is one backend: one device, one in-order HIP stream, the weights it has prepared. It stands in for
 * xtg::OpenClBackend (engine/include/xtg/opencl.h:22-63) and for the CPU kernel entry points the Dory pack calls
 * (engine/include/xtg/kernels.h:27-49, engine/include/xtg/kv.h:21-79). Conventions follow the reference's
 * plugin ABI (npu/xtg_npu.h:14-47): opaque handles, a NULL handle on failure, `int` return codes (0 success,
 * -1 failure) with the message written into `err` (err_len bytes, NUL-terminated), JSON from info(). No call
 * throws or aborts across this boundary.
 *
 * Device-resident calls only queue work on the backend's stream, like the OpenCL backend's in-order queue
 * (opencl.h:16-21); xtg_hip_read() and xtg_hip_finish() wait for it. Pointers documented as "device" are
 * addresses from xtg_hip_alloc() (or any device allocation on the same device); "host" pointers are ordinary
 * memory. One backend is used from one thread at a time (packs/dory: one engine thread, server/runtime.h:1-3).
 */
#ifndef XTG_HIP_H
#define XTG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XTG_HIP_ABI_VERSION 2

typedef struct xtg_hip xtg_hip;
typedef struct xtg_hip_kv xtg_hip_kv;

/* An NVFP4 weight [n_out][k] in ModelOpt's layout: E2M1 codes two per byte (element 2j in the low nibble of byte
 * j), one E4M3 scale per 16 inputs, one FP32 scale for the tensor; w[n][j] = e2m1 * e4m3(scale[n][j/16]) * global.
 * Field for field the same as xtg::Nvfp4Weight (engine/include/xtg/kernels.h:13-20), so an array of those can be
 * passed as is. codes / scales are host pointers; they key the prepared device copy (as opencl.cpp:489-492). */
typedef struct xtg_nvfp4 {
  const uint8_t* codes;   /* [n_out][k / 2] */
  const uint8_t* scales;  /* [n_out][k / 16] */
  float global;
  int n_out, k;
} xtg_nvfp4;

/* A BF16 weight [n_out][k], row-major (a BF16 checkpoint's LM head): field for field xtg::Bf16Weight
 * (engine/include/xtg/kernels.h:22-25). data is a host pointer; it keys the prepared device copy. */
typedef struct xtg_bf16 {
  const uint16_t* data;   /* [n_out][k] BF16 bits */
  int n_out, k;
} xtg_bf16;

enum { XTG_X_F32 = 0, XTG_X_BF16 = 1 };   /* activation element type of the device matmul */
enum { XTG_KV_BF16 = 0, XTG_KV_FP8 = 1 }; /* xtg::KvDtype (engine/include/xtg/kv.h:18) */
/* The recurrent sublayers' KV mode (the pack's kv_mode option, packs/dory/dory.cpp:150-151): per_loop keeps one cache
 * per loop; last_loop keeps one cache that only the last loop writes (dory.cpp:534-537). */
enum { XTG_KV_PER_LOOP = 0, XTG_KV_LAST_LOOP = 1 };

/* ------------------------------------------------------------------------------------------------ backend */

/* Replaces OpenClBackend::OpenClBackend() (opencl.h:28). options: JSON, may be NULL or empty; keys: "device"
 * (HIP device index, default 0). NULL on failure, the reason in err. */
xtg_hip* xtg_hip_open(const char* options, char* err, int err_len);
/* Replaces ~OpenClBackend (opencl.h:29): waits for queued work, frees every device buffer the backend owns. */
void xtg_hip_close(xtg_hip* h);
/* Replaces device_name() / weight_bytes() (opencl.h:36-37): {"abi", "device", "arch", "cus", "hbm_bytes",
 * "weight_bytes", "weights"} as JSON. Returns the length written (without the NUL), or -1. */
int xtg_hip_info(xtg_hip* h, char* out, int out_len);
/* The backend's hipStream_t, for callers that time or order their own work against it. */
void* xtg_hip_stream(xtg_hip* h);

/* --------------------------------------------------------------------------------------------- NVFP4 path */

/* Replaces OpenClBackend::prepare(const Nvfp4Weight&) (opencl.h:32, opencl.cpp:489-515): copy the weight to the
 * device in the GEMV tile layout. Idempotent, keyed by w->codes. k % 16 == 0 and n_out > 0 are required. */
int xtg_hip_prepare_nvfp4(xtg_hip* h, const xtg_nvfp4* w, char* err, int err_len);
/* Drops the device copy prepared for `codes` (a weight whose host memory is about to be freed or reused). The
 * reference frees its device weights only with the backend (opencl.cpp:349-353); callers that recycle host
 * buffers need this to keep the codes-pointer key unambiguous. 0 also when nothing was prepared for it; -1 while a
 * Dory session runs on the weight. */
int xtg_hip_release_nvfp4(xtg_hip* h, const uint8_t* codes, char* err, int err_len);
/* The device tile layout prepare() made for the weight keyed by `codes` (16 rows x 128 inputs per 1152-byte tile:
 * 1024 bytes of codes, lane l's 16 at 16 l, then lane l's two scales at 1024 + 2 l), copied to host memory; bytes
 * must be ceil(n/16) * ceil(k/128) * 1152. No counterpart in the reference (whose OpenCL repack is internal): for
 * checking the device repack of a checkpoint's arrays. */
int xtg_hip_nvfp4_tiles(xtg_hip* h, const uint8_t* codes, void* out, size_t bytes, char* err, int err_len);
/* Replaces xtg::matmul_nvfp4(ThreadPool&, ws, x, m, ys) (kernels.h:27-30, kernels.cpp:84-138) and the host
 * OpenClBackend::matmul (opencl.h:34, opencl.cpp:523-601): y_i[m][n_out_i] = x[m][k] * W_i^T for n_w weights
 * sharing k; x and every ys[i] are host memory; synchronous. Prepares weights not seen before. m >= 1 (rows are
 * processed in passes of up to 512: the GEMV for 1-8 rows, the matrix-core GEMM above). */
int xtg_hip_matmul_nvfp4(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const float* x, int m, float* const* ys,
                         char* err, int err_len);
/* Replaces OpenClBackend::matmul(ws, Mem x, m, Mem y, y_offset) (opencl.h:54-55, opencl.cpp:694-754): the n_w
 * projections of the device input x ([m][k], FP32 or BF16 per x_dtype) into consecutive [m][n_out_i] blocks of
 * the device output y starting at y_offset floats. Queued; 1 <= m <= 4096 (1-8 rows: the GEMV, which reads the rows
 * as they are; more: the GEMM on a prepared operand), n_w <= 4 per call (the fused q/k/v/g and gate/up of the Dory
 * sublayers). x must be 16-byte aligned. The GEMM keeps ~22 bits of each activation (two f16 parts); with
 * XTG_GEMM_PARTS=1 in the environment (read at each call) it takes one f16 part, about 1.4-1.6x faster at ~2e-4
 * relative error, the precision class of the reference's FP16 GPU prefill GEMM (opencl.cpp:232-269). One or two
 * BF16 rows run on the block-scaled FP4 x FP8 matrix op (no dequantisation; each BF16 input split exactly into two
 * E4M3 parts); XTG_GEMV_MX=0 in the environment (read once) keeps them on the f16 matrix op, for comparison. */
int xtg_hip_matmul_nvfp4_dev(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const void* x, int x_dtype, int m, float* y,
                             size_t y_offset, char* err, int err_len);

/* The device matmul in its two steps, for callers that reuse one activation operand or produce it themselves
 * (no counterpart in the reference, whose kernels read FP32 x directly): xtg_hip_x_operand_bytes(k) bytes of
 * device memory hold the matrix-core form of 8 rows of x, and m rows take ceil(m / 8) such groups back to back;
 * xtg_hip_prep_x fills it (queued) and xtg_hip_matmul_nvfp4_op runs the projections on it with the same output
 * convention as the call above (1 <= m <= 4096). */
size_t xtg_hip_x_operand_bytes(int k);
int xtg_hip_prep_x(xtg_hip* h, const void* x, int x_dtype, int m, int k, void* op, char* err, int err_len);
int xtg_hip_matmul_nvfp4_op(xtg_hip* h, const xtg_nvfp4* ws, int n_w, const void* op, int m, float* y, size_t y_offset,
                            char* err, int err_len);

/* ---------------------------------------------------------------------------------------------- BF16 path */

/* Replaces OpenClBackend::prepare(const Bf16Weight&) (opencl.h:33, opencl.cpp:516-521): copy the weight to the
 * device in the GEMV tile layout. Idempotent, keyed by w->data. n_out > 0 and k % 4 == 0 (as opencl.cpp:519). */
int xtg_hip_prepare_bf16(xtg_hip* h, const xtg_bf16* w, char* err, int err_len);
/* Drops the device copy prepared for `data` (0 also when there is none; -1 while a Dory session runs on it). */
int xtg_hip_release_bf16(xtg_hip* h, const uint16_t* data, char* err, int err_len);
/* Replaces xtg::matmul_bf16(ThreadPool&, w, x, m, y) (kernels.h:31, kernels.cpp:140-155) and the host
 * OpenClBackend::matmul(const Bf16Weight&, x, m, y) (opencl.h:35, opencl.cpp:602-628): y[m][n_out] =
 * x[m][k] * W^T with FP32 products and sums; x, y host memory; synchronous; m >= 1 (8 rows per pass). */
int xtg_hip_matmul_bf16(xtg_hip* h, const xtg_bf16* w, const float* x, int m, float* y, char* err, int err_len);
/* Replaces OpenClBackend::matmul(const Bf16Weight&, Mem x, m, Mem y) (opencl.h:56, opencl.cpp:755-780): device
 * x ([m][k], FP32 or BF16 per x_dtype) into device y [m][n_out] from y_offset floats. Queued; 1 <= m <= 8. */
int xtg_hip_matmul_bf16_dev(xtg_hip* h, const xtg_bf16* w, const void* x, int x_dtype, int m, float* y,
                            size_t y_offset, char* err, int err_len);

/* ------------------------------------------------------------------------------------------- KV caches */

/* Replaces xtg::KvCache(kv_heads, head_dim, slots, ring, dtype) (kv.h:24, kv.cpp:42-63): ring > 0 makes a ring of
 * `ring` slots (slot = position mod ring), else a linear cache of `slots` positions, in device memory: BF16
 * (XTG_KV_BF16) or E4M3 codes with one FP32 scale per (position, KV head) (XTG_KV_FP8). Every slot starts empty.
 * NULL on failure. */
xtg_hip_kv* xtg_hip_kv_create(xtg_hip* h, int kv_heads, int head_dim, int64_t slots, int ring, int dtype, char* err,
                              int err_len);
void xtg_hip_kv_destroy(xtg_hip* h, xtg_hip_kv* kv);
/* Replaces KvCache::store (kv.h:35, kv.cpp:75-112): rows of positions pos .. pos + n - 1 from device FP32 k, v
 * [n][kv_heads][head_dim], rounded to BF16 (nearest even), or for FP8 scaled by amax / 448 of each (row, head)
 * and rounded as kv.cpp:19-40 does; a ring keeps the last `ring` rows; queued. A linear cache refuses positions
 * beyond its capacity ("KV cache full"). */
int xtg_hip_kv_store(xtg_hip* h, xtg_hip_kv* kv, int64_t pos, int n, const float* k, const float* v, char* err,
                     int err_len);
/* Replaces KvCache::load (kv.h:37, kv.cpp:114-138): FP32 K and V rows of head `head` for positions p0 .. p1 - 1
 * into host k, v [p1 - p0][head_dim]; waits for queued work. */
int xtg_hip_kv_load(xtg_hip* h, const xtg_hip_kv* kv, int head, int64_t p0, int64_t p1, float* k, float* v, char* err,
                    int err_len);
/* Replaces KvCache::save / restore / release (kv.h:45-48): the whole cache (K, V, FP8 scales and slot positions,
 * in the device layout) as xtg_hip_kv_bytes() host bytes and back; release empties every slot. */
int64_t xtg_hip_kv_bytes(xtg_hip* h, const xtg_hip_kv* kv);
int xtg_hip_kv_save(xtg_hip* h, const xtg_hip_kv* kv, void* out, size_t bytes, char* err, int err_len);
int xtg_hip_kv_restore(xtg_hip* h, xtg_hip_kv* kv, const void* in, size_t bytes, char* err, int err_len);
int xtg_hip_kv_release(xtg_hip* h, xtg_hip_kv* kv, char* err, int err_len);
/* GpuDorySession::snapshot / restore's per-ring device copies (dory.cpp:1231-1273): the whole state of src (data,
 * FP8 scales, slot positions) into dst, a cache of the same shape, ring size and dtype; device to device, queued. */
int xtg_hip_kv_copy(xtg_hip* h, const xtg_hip_kv* src, xtg_hip_kv* dst, char* err, int err_len);

/* ------------------------------------------------------------------------------------------- attention */

/* xtg::AttnArgs (kv.h:67-78), field for field, with device pointers and a device cache. */
typedef struct xtg_attn_args {
  int n_q;
  int64_t pos0;
  int heads, kv_heads, head_dim;
  int window;
  float scale;
  const float* q;   /* [n_q][heads][head_dim] */
  const float* k;   /* [n_q][kv_heads][head_dim]: this call's keys, FP32, not yet stored */
  const float* v;
  const xtg_hip_kv* cache;
  float* out;       /* [n_q][heads][head_dim] */
} xtg_attn_args;
/* Replaces xtg::attention(ThreadPool&, const AttnArgs&) (kv.h:79, kv.cpp:166-286): causal GQA attention of the
 * call's n_q rows over the cached positions before pos0 plus the call's own keys; window > 0 limits a row at t to
 * keys t - window + 1 .. t. The cache is read only; which slots a row sees is decided from the positions stored
 * in them (for a ring: npu/xtg_npu.cpp:236-258). Queued. head_dim 64, 128 or 256, at most 8 q heads per KV head. */
int xtg_hip_attention(xtg_hip* h, const xtg_attn_args* a, char* err, int err_len);
/* No counterpart in the reference: xtg_hip_attention for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and results; it
 * allocates nothing: the split partials go to one fixed device array of XTG_HIP_ATTN_SCRATCH_BYTES per device, held
 * from the library's load until the process ends (profiling events are made only while xtg_hip_profile is on). A
 * call whose partials exceed the array fails (-1, the sizes in err) before anything is queued: decode and verify
 * calls fit (8 rows over 8 KV heads of 128 take about 2 MB), long prefill chunks may not. The array belongs to the
 * first backend (xtg_hip handle) that calls this on the device, until that backend is closed; a call from another
 * backend on the same device meanwhile fails (-1), since their calls would race on the one array. Calls queued on
 * the owning backend's stream run in order; each rewrites every partial it reads. */
#define XTG_HIP_ATTN_SCRATCH_BYTES (16u << 20)
int xtg_hip_attention_noalloc(xtg_hip* h, const xtg_attn_args* a, char* err, int err_len);

/* ----------------------------------------------------------------------------------------- row kernels */

/* The Q/K producer of an attention sublayer (packs/dory/dory.cpp:482-490; the OpenCL rope_norm, dory.cpp:728-746):
 * NeoX RoPE of q [m][heads][head_dim] and k [m][kv_heads][head_dim] at positions pos0 + row (inv_freq as
 * engine/src/kernels.cpp:191-201), justnorm per head, then q times qscale [heads * head_dim] (NULL: no scale);
 * in place, queued. */
int xtg_hip_qk_rope_norm(xtg_hip* h, float* q, float* k, int m, int heads, int kv_heads, int head_dim, int64_t pos0,
                         float theta, const float* qscale, char* err, int err_len);
/* xtg::slerp_residual (kernels.h:43, kernels.cpp:177-189; OpenCL slerp dory.cpp:680-696): x = justnorm(ya + lr *
 * (yb - ya)), ya = justnorm(x), yb = justnorm(o), per row of width; in place, queued. */
int xtg_hip_slerp_residual(xtg_hip* h, float* x, const float* o, const float* lr, int rows, int width, char* err,
                           int err_len);
/* swiglu_scaled then justnorm (kernels.h:48, kernels.cpp:225-234, dory.cpp:474-475; OpenCL swiglu_norm
 * dory.cpp:698-711): g = justnorm(silu(g * sg) * (u * su)); in place, queued. */
int xtg_hip_swiglu_norm(xtg_hip* h, float* g, const float* u, const float* sg, const float* su, int rows, int width,
                        char* err, int err_len);
/* The attention output gate (dory.cpp:510-515; OpenCL gate_norm dory.cpp:713-726): att = justnorm(att *
 * sigmoid(gate * gs)) over each row; in place, queued. */
int xtg_hip_gate_norm(xtg_hip* h, float* att, const float* gate, const float* gs, int rows, int width, char* err,
                      int err_len);
/* The loop entry / exit norms (dory.cpp:532-541; OpenCL add_norm dory.cpp:669-678): out = justnorm(a + b), or
 * justnorm(a) when b is NULL; out may be a; queued. */
int xtg_hip_add_norm(xtg_hip* h, const float* a, const float* b, float* out, int rows, int width, char* err,
                     int err_len);
/* xtg::argmax (engine/include/xtg/sampler.h:29, engine/src/sampler.cpp:8-13), greedy decoding's token, per row of
 * device logits [rows][n] into device out [rows] (int32): the first index of the largest value; NaNs never win, and
 * a NaN in element 0 gives 0, as the reference's scan does. Queued. Up to 8 rows of more than 4096 logits use
 * scratch memory that the first call of a shape sizes: make that call before a graph capture. */
int xtg_hip_argmax(xtg_hip* h, const float* logits, int rows, int n, int32_t* out, char* err, int err_len);
/* xtg::SamplingParams (engine/include/xtg/sampler.h:11-16), field for field. */
typedef struct xtg_sampling {
  float temperature; /* 0: greedy */
  float top_p;
  int top_k;         /* 0: off */
  float min_p;
} xtg_sampling;
/* xtg::Sampler::sample (engine/src/sampler.cpp:40-94) per row of device logits [rows][n] (rows <= 8) into device
 * out [rows] (int32). The random draw stays with the caller's generator: u [rows] (host) holds, per row, the
 * value the reference's std::uniform_real_distribution<double>(0, total) scales by the total, i.e.
 * std::generate_canonical<double, 53>(rng) from the Sampler's std::mt19937_64 (one draw per sampled row, none when
 * temperature <= 0, which is argmax). Candidates are ordered by weight then index over the whole row, as the
 * reference orders them wherever its result is defined. Queued; the first call of a shape sizes scratch memory
 * (make it before a graph capture). */
int xtg_hip_sample(xtg_hip* h, const float* logits, int rows, int n, const xtg_sampling* p, const double* u,
                   int32_t* out, char* err, int err_len);

/* ----------------------------------------------------------------------------------- Dory decode step */

/* The looped-nGPT model's sublayer kinds (packs/dory/dory.cpp:38) and shape (dory.cpp:45-56). */
enum { XTG_DORY_MLP = 0, XTG_DORY_SLIDING = 1, XTG_DORY_FULL = 2 };
typedef struct xtg_dory_config {
  int hidden, ffn, heads, kv_heads, head_dim, vocab;
  int n_in, n_rec, n_out, loops;   /* input / recurrent / output sublayers; recurrent passes */
  int window, ring_slots;          /* sliding window and the ring size of a sliding sublayer's cache */
  int64_t context;                 /* capacity of a full-attention cache */
  float theta_sliding, theta_full; /* RoPE theta per kind */
  int kv_dtype;                    /* XTG_KV_BF16 or XTG_KV_FP8 (dory.cpp:141, 159-161) for every cache */
  int kv_mode;                     /* XTG_KV_PER_LOOP or XTG_KV_LAST_LOOP */
} xtg_dory_config;
/* One physical sublayer (dory.cpp:332-364) with the scale vectors already folded as the model constructor does
 * (qscale = (sqk * sqrt(d) / init_range)^2, gscale likewise, sg / su times sqrt(hidden), lr = |alpha * alpha_init /
 * init_range|). Weights are host NVFP4 tensors (prepared to the device by create), vectors host FP32. */
typedef struct xtg_dory_layer {
  int kind;
  xtg_nvfp4 q, k, v, g, o;      /* attention */
  xtg_nvfp4 gate, up, down;     /* MLP */
  const float* qscale;          /* [heads * head_dim] */
  const float* gscale;          /* [heads * head_dim] */
  const float* sg;              /* [ffn] */
  const float* su;              /* [ffn] */
  const float* lr;              /* [hidden] */
} xtg_dory_layer;
typedef struct xtg_hip_dory xtg_hip_dory;
/* Replaces the DoryModel constructor's weight preparation (dory.cpp:365-371) and the GpuDorySession constructor
 * (dory.cpp:1043-1084): prepares every weight and the NVFP4 LM head [vocab][hidden] (head may be NULL when a BF16
 * head follows through xtg_hip_dory_head_bf16), uploads the vectors and logit_scale [vocab], creates the caches
 * (kv_dtype; sliding sublayers: rings of ring_slots) and, per RoPE theta, the cosines and sines of every position
 * below context (context x head_dim / 2 x 8 bytes of device memory each). NULL on failure. The host weights must
 * stay alive and unchanged while the session exists (they key the prepared copies). */
xtg_hip_dory* xtg_hip_dory_create(xtg_hip* h, const xtg_dory_config* c, const xtg_dory_layer* layers,
                                  const xtg_nvfp4* head, const float* logit_scale, char* err, int err_len);
void xtg_hip_dory_destroy(xtg_hip_dory* d);
/* A BF16 LM head [vocab][hidden] in place of the NVFP4 one: a BF16 checkpoint's lm_head.weight (dory.cpp:325),
 * the head the resident GPU session runs (dory.cpp:1203, opencl.h:56). The logits become (x * W^T) * logit_scale
 * with FP32 products and sums (kernels.cpp:140-155). Prepared on the call; not during a graph capture. */
int xtg_hip_dory_head_bf16(xtg_hip_dory* d, const xtg_bf16* head, char* err, int err_len);
/* Replaces GpuDorySession::run_chunk + the head of forward (dory.cpp:1150-1214; CPU dory.cpp:520-578) for one
 * chunk of m <= 512 rows: from the hidden rows x [m][hidden] (device, the embedding rows) at positions pos0 ..
 * pos0 + m - 1 to logits [m][vocab] (device, times logit_scale); each attention sublayer's cache gains the chunk's
 * keys. Up to 8 rows (a decode or verify step) run the fused decode kernels; more run the prefill kernels (the
 * matrix-core GEMM, many-row attention). Queued: capturable into a graph (xtg_hip_graph_*) once the call has run
 * with the same m. */
int xtg_hip_dory_forward(xtg_hip_dory* d, const float* x, int m, int64_t pos0, float* logits, char* err, int err_len);
/* Which rows get logits (xtg::Logits, engine/include/xtg/model.h:28). */
enum { XTG_LOGITS_NONE = 0, XTG_LOGITS_LAST = 1, XTG_LOGITS_ALL = 2 };
/* Replaces DorySession::forward's chunk loop (dory.cpp:554-578): n rows of x [n][hidden] (device) at positions
 * pos0 .. pos0 + n - 1 in chunks of up to 512 rows (the prefill chunk), with logits (device, times logit_scale)
 * for every row ([n][vocab], XTG_LOGITS_ALL), the last row ([vocab], XTG_LOGITS_LAST) or none (logits may be
 * NULL). Queued. */
int xtg_hip_dory_prefill(xtg_hip_dory* d, const float* x, int n, int64_t pos0, int want, float* logits, char* err,
                         int err_len);
/* Replaces DorySession / GpuDorySession::snapshot and restore (dory.cpp:591-614, 1231-1273): device copies of
 * every sliding sublayer's ring into snapshot slot `slot` (0..63; its storage is made on first use), and back.
 * Global caches are not copied: keys written past the restored position are masked by position. The caller keeps
 * the position (the reference's n_). Queued. */
int xtg_hip_dory_snapshot(xtg_hip_dory* d, int slot, char* err, int err_len);
int xtg_hip_dory_restore(xtg_hip_dory* d, int slot, char* err, int err_len);
/* The cache of attention sublayer `attn` (counted over attention sublayers) for loop `inst`, e.g. to fill a
 * context with xtg_hip_kv_store. NULL when there is none. */
xtg_hip_kv* xtg_hip_dory_cache(xtg_hip_dory* d, int attn, int inst);

/* ------------------------------------------------------------------------------------- device buffers */

/* Replaces OpenClBackend::alloc / release / write / read / copy / finish (opencl.h:40-45). write() is blocking
 * (src may be reused on return), read() waits for all queued work, copy() is queued. */
int xtg_hip_alloc(xtg_hip* h, size_t bytes, void** out, char* err, int err_len);
void xtg_hip_release(xtg_hip* h, void* mem);
int xtg_hip_write(xtg_hip* h, void* mem, size_t offset, const void* src, size_t bytes, char* err, int err_len);
int xtg_hip_read(xtg_hip* h, const void* mem, size_t offset, void* dst, size_t bytes, char* err, int err_len);
int xtg_hip_copy(xtg_hip* h, const void* src, size_t src_offset, void* dst, size_t dst_offset, size_t bytes,
                 char* err, int err_len);
int xtg_hip_finish(xtg_hip* h, char* err, int err_len);

/* ------------------------------------------------------------------------------------------------- graphs */

/* No counterpart in the reference (its OpenCL queue replays nothing): HIP graphs over the backend's stream. Every
 * device call queued between begin and end is captured into one graph instead of running; launch replays it on the
 * stream. Weights must be prepared and scratch sized before the capture (run the calls once first); blocking calls
 * fail during a capture. A graph replays its calls exactly as captured, arguments included: a captured decode step
 * is the step at its captured position (RoPE angles, cache slots and scan plan are arguments), so a decode loop
 * captures one graph per position or runs eagerly. While any graph exists
 * the backend frees no device memory a graph may address: scratch that a later, larger call outgrows, and weights,
 * buffers and caches released meanwhile, are kept until the last graph is destroyed (the memory of the caller's
 * own buffers is kept, but their contents are the caller's). `name` (may be NULL) is the graph's entry in the
 * profile report, where a profiled replay is timed as a whole. */
typedef struct xtg_hip_graph xtg_hip_graph;
int xtg_hip_graph_begin(xtg_hip* h, char* err, int err_len);
int xtg_hip_graph_end(xtg_hip* h, const char* name, xtg_hip_graph** out, char* err, int err_len);
int xtg_hip_graph_launch(xtg_hip* h, xtg_hip_graph* g, char* err, int err_len);
void xtg_hip_graph_destroy(xtg_hip* h, xtg_hip_graph* g);

/* ---------------------------------------------------------------------------------------------- profiling */

/* Replaces the XTG_GPU_PROFILE switch of the OpenCL backend (opencl.cpp:293-315, :391-392): with enable != 0
 * every kernel the backend queues is bracketed by two events on its stream; enable == 2 also keeps every launch's
 * time in queue order for the report. */
int xtg_hip_profile(xtg_hip* h, int enable, char* err, int err_len);
/* Waits for queued work and writes {"kernels": {name: {"calls": n, "ms": total}}} for the launches recorded since
 * the last report (names as rocprof prints them, without the namespace), with "launches": [[name, ms], ...] in
 * queue order after enable == 2, then starts over. Returns the length (without the NUL), or -1; a report longer
 * than out_len is cut (and its records are gone). */
int xtg_hip_profile_report(xtg_hip* h, char* out, int out_len);

/* ------------------------------------------------------------------------------------------------ probes */

/* The device probe's streaming read (tests/gpu_probe.cpp:59-66, readsum: a buffer summed in 16-byte loads, one
 * partial per work-group): every byte of src (device, 16-byte aligned, a multiple of 16 bytes) read once and
 * XOR-folded into out (device, xtg_hip_read_probe_partials(bytes) uint32 partials, one per work-group of 256 threads
 * with 8 loads each). Queued. Profiled by xtg_hip_profile like any kernel: the read roofline of this device at a
 * given size. */
size_t xtg_hip_read_probe_partials(size_t bytes);
int xtg_hip_read_probe(xtg_hip* h, const void* src, size_t bytes, uint32_t* out, char* err, int err_len);

#ifdef __cplusplus
}
#endif
#endif
