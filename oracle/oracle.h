/* CPU oracle for the xtier-go decode kernel layer.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference engine's CPU kernels, used as the
 * checker for the HIP kernels. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the checker or the CPU baseline -- never as the thing measured or shipped. The HIP library
 * never links or calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to the reference root). Pinning
 * (what independent check each function is held to) is listed per function; tests/test_oracle_*.py run them.
 *
 * Threading: functions that take `threads` split independent outputs over OpenMP threads; every output is
 * computed by one thread in a fixed order, so results do not depend on the thread count.
 */
#ifndef XTG_ORACLE_H
#define XTG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- number formats: engine/include/xtg/fp.h:10-41, engine/src/fp.cpp:12-49, engine/src/kv.cpp:19-40 --- */
float xo_bf16_to_f32(uint16_t h);            /* fp.h:10-15 */
uint16_t xo_f32_to_bf16(float f);            /* fp.h:18-24, RNE, NaN kept quiet */
float xo_e4m3_to_f32(uint8_t b);             /* fp.cpp:12-28 table */
uint8_t xo_f32_to_e4m3(float f);             /* fp.cpp:30-49, RNE by search, saturate to 448 */
uint8_t xo_e4m3_bits(float x);               /* kv.cpp:19-40, the KV cache's bit-level RNE */
float xo_e2m1(int code);                     /* fp.h:37-39 */

/* --- NVFP4 weights: engine/include/xtg/kernels.h:13-20 (same field order as xtg::Nvfp4Weight) --- */
typedef struct xo_nvfp4 {
  const uint8_t* codes;   /* [n_out][k/2], element 2j in the low nibble of byte j */
  const uint8_t* scales;  /* [n_out][k/16] E4M3 */
  float global;
  int n_out, k;
} xo_nvfp4;

void xo_nvfp4_row(const xo_nvfp4* w, int n, float* out);          /* kernels.cpp:34-45 */
/* kernels.cpp:84-138: m <= 2 decode branch (dot_nvfp4 :48-60), m > 2 prefill branch (nvfp4_row + dot_f32).
 * ys[i] holds m * ws[i].n_out floats. Returns 0, or -1 when the widths differ / k % 16 != 0 (kernels.cpp:86-88). */
int xo_matmul_nvfp4(const xo_nvfp4* ws, int n_w, const float* x, int m, float* const* ys, int threads);
int xo_matmul_bf16(const uint16_t* w, int n_out, int k, const float* x, int m, float* y,
                   int threads);   /* kernels.cpp:140-155 */

/* --- row kernels: engine/src/kernels.cpp:157-234 --- */
void xo_bf16_row(const uint16_t* table, int64_t row, int width, float* out);               /* :157-160 */
void xo_justnorm(float* x, int rows, int width);                                          /* :162-175 */
void xo_slerp_residual(float* a, const float* b, const float* lr, int rows, int width);   /* :177-189 */
void xo_rope(float* x, int rows, int heads, int head_dim, int64_t pos0, float theta);     /* :191-223 */
void xo_swiglu_scaled(float* g, const float* u, const float* sg, const float* su, int rows, int w); /* :225-234 */
/* The RoPE table the reference GPU session uploads (packs/dory/dory.cpp:1159-1171): cs[r][i] = cos, then
 * cs[m + r][i] = sin, for rows at pos0 + r. */
void xo_rope_table(float* cs, int m, int head_dim, int64_t pos0, float theta);

/* --- sublayer compositions of packs/dory/dory.cpp --- */
/* :510-515: att[r][j] *= 1 / (1 + exp(-gate[r][j] * gs[j])), then justnorm of each row */
void xo_gate_norm(float* att, const float* gate, const float* gs, int rows, int width);
/* :532-541: out = justnorm(a + b) (b non-NULL) or justnorm(a); out may alias a */
void xo_add_norm(const float* a, const float* b, float* out, int rows, int width);
int xo_argmax(const float* x, int n);                                                      /* sampler.cpp:8-13 */
int xo_sample(const float* logits, int n, float temperature, float top_p, int top_k, float min_p, double u,
              double* margin);                                                             /* sampler.cpp:40-94 */

/* --- Q/K producer: packs/dory/dory.cpp:481-490 (RoPE q and k, justnorm per head, q *= qscale) --- */
void xo_qk_produce(float* q, float* k, int m, int heads, int kv_heads, int head_dim, int64_t pos0, float theta,
                   const float* qscale);

/* --- KV cache: engine/include/xtg/kv.h:21-62, engine/src/kv.cpp:42-149 --- */
typedef struct xo_kv xo_kv;
enum { XO_KV_BF16 = 0, XO_KV_FP8 = 1 };
xo_kv* xo_kv_create(int kv_heads, int head_dim, int64_t slots, int ring, int dtype);   /* kv.cpp:42-63 */
void xo_kv_free(xo_kv* c);
int64_t xo_kv_slots(const xo_kv* c);
int xo_kv_store(xo_kv* c, int64_t pos, int n, const float* k, const float* v);           /* kv.cpp:75-112 */
void xo_kv_load(const xo_kv* c, int h, int64_t p0, int64_t p1, float* k, float* v);     /* kv.cpp:114-138 */
/* raw storage (slot-major [slots][kv_heads][head_dim], 2 or 1 bytes per element; FP8 scales [slots][kv_heads]) */
const void* xo_kv_kdata(const xo_kv* c);
const void* xo_kv_vdata(const xo_kv* c);
const float* xo_kv_kscale(const xo_kv* c);
const float* xo_kv_vscale(const xo_kv* c);

/* --- attention: engine/include/xtg/kv.h:64-79, engine/src/kv.cpp:153-286 --- */
typedef struct xo_attn_args {
  int n_q;
  int64_t pos0;
  int heads, kv_heads, head_dim;
  int window;
  float scale;
  const float* q;   /* [n_q][heads][head_dim] */
  const float* k;   /* [n_q][kv_heads][head_dim] this call's keys */
  const float* v;
  const xo_kv* cache;
  float* out;       /* [n_q][heads][head_dim] */
} xo_attn_args;
/* `pool_size` plays the role of ThreadPool::size() in the split heuristic (kv.cpp:174-177); the work runs on
 * `threads` OpenMP threads. Returns -1 on an unsupported head grouping (kv.cpp:168-169). */
int xo_attention(const xo_attn_args* a, int pool_size, int threads);
/* Ring attention by stored slot positions, the NPU plugin's mask (npu/xtg_npu.cpp:236-258): a query row at
 * position p sees ring slot s iff 0 <= slot_pos[s] < pos0 and p - slot_pos[s] < window (window > 0), plus this
 * call's rows j <= i with i - j < window. One pass per (row, head) over all slots in slot order, FP32 online
 * softmax over tiles of 64 slots. */
int xo_attention_slots(const xo_attn_args* a, const int64_t* slot_pos, int threads);

/* --- the Dory decode step: packs/dory/dory.cpp:467-578 --- */
enum { XO_MLP = 0, XO_SLIDING = 1, XO_FULL = 2 };   /* dory.cpp:38 */
typedef struct xo_dory_layer {
  int kind;
  xo_nvfp4 q, k, v, g, o;          /* attention sublayer */
  xo_nvfp4 gate, up, down;         /* MLP sublayer */
  const float* qscale;             /* [heads * head_dim], folded as dory.cpp:354-357 */
  const float* gscale;             /* [heads * head_dim] */
  const float* sg;                 /* [ffn], folded (dory.cpp:342-345) */
  const float* su;
  const float* lr;                 /* [hidden], |alpha * scale| (dory.cpp:363) */
} xo_dory_layer;
typedef struct xo_dory_config {
  int hidden, ffn, heads, kv_heads, head_dim, vocab;
  int n_in, n_rec, n_out, loops;   /* input / recurrent / output sublayers; recurrent passes */
  int window, ring_slots;          /* sliding window and its ring size */
  int64_t context;                 /* linear cache capacity */
  float theta_sliding, theta_full;
  int kv_dtype;                    /* XO_KV_BF16 | XO_KV_FP8 for every cache (dory.cpp:141, 159-161) */
  int kv_mode;                     /* XO_KV_PER_LOOP | XO_KV_LAST_LOOP (dory.cpp:150-151) */
} xo_dory_config;
enum { XO_KV_PER_LOOP = 0, XO_KV_LAST_LOOP = 1 };
typedef struct xo_dory xo_dory;
/* Layers and vectors are borrowed (they must outlive the model). KV modes (dory.cpp:436-447, 530-537): per_loop, a
 * recurrent attention sublayer keeps one cache per loop; last_loop, one cache that only the last loop writes (every
 * loop attends to it plus the chunk's own keys). */
xo_dory* xo_dory_create(const xo_dory_config* c, const xo_dory_layer* layers, const xo_nvfp4* head,
                        const float* logit_scale);
void xo_dory_free(xo_dory* d);
/* The cache of attention sublayer `attn` (counted over attention sublayers), loop instance `inst`. */
xo_kv* xo_dory_cache(xo_dory* d, int attn, int inst);
/* A BF16 LM head [vocab][hidden] (borrowed) in place of the NVFP4 one: dory.cpp:325, 401-402 */
void xo_dory_head_bf16(xo_dory* d, const uint16_t* w);
/* dory.cpp:520-544 run_chunk from the hidden rows x [m][hidden] (the embedding rows) at positions pos0 .., then the
 * head for every row times logit_scale (dory.cpp:566-576): logits [m][vocab]; the caches gain the chunk's keys. */
int xo_dory_forward(xo_dory* d, const float* x, int m, int64_t pos0, float* logits, int threads);

#ifdef __cplusplus
}
#endif
#endif
