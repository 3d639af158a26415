#include "dory.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <utility>

#include "common.hpp"

namespace xtg::hip {

namespace {
constexpr int kChunkRows = 512;   // rows of one run_chunk: the reference's prefill chunk (dory.cpp:145-148)
constexpr int kMaxSnapshots = 64;
}

namespace {
// 2^e with |v 2^e| <= 2^14 for every |v| <= bound (an f16 operand part's headroom; 1 for bound 0)
float operand_factor(double bound) {
  if (!(bound > 0.0)) return 1.f;
  int p = 0;
  (void)std::frexp(bound, &p);   // bound < 2^p
  return std::ldexp(1.f, std::max(-60, std::min(60, 14 - p)));
}

// The largest |w| of an NVFP4 weight: |global| * 6 (E2M1's largest) * its largest E4M3 scale (the codes' order
// follows the magnitudes'; a NaN code counts as 448, E4M3's largest finite value).
double max_abs_weight(const xtg_nvfp4& w) {
  int top = 0;
  const size_t n = size_t(w.n_out) * size_t(w.k / 16);
  for (size_t i = 0; i < n; ++i) top = std::max(top, int(w.scales[i] & 0x7f));
  const int e = top >> 3, m = top & 7;
  const double scale = top >= 0x7e ? 448.0 : e == 0 ? std::ldexp(double(m), -9) : std::ldexp(1.0 + m / 8.0, e - 7);
  return std::fabs(double(w.global)) * 6.0 * scale;
}
}  // namespace

float* DorySession::upload(const float* v, size_t n) {
  XTG_CHECK(v, "dory: a per-layer vector is NULL");
  float* p = static_cast<float*>(b_.alloc(n * sizeof(float)));
  b_.write(p, 0, v, n * sizeof(float));
  owned_.push_back(p);
  return p;
}

void DorySession::prepare(const xtg_nvfp4& w) {
  const bool fresh = w.codes && !b_.has_weight(w.codes);
  b_.prepare(w);
  b_.hold(w.codes, fresh);
  held_.push_back(w.codes);
}

DorySession::DorySession(Backend& b, const xtg_dory_config& c, const xtg_dory_layer* layers, const xtg_nvfp4& head,
                         const float* logit_scale)
    : b_(b), c_(c), head_(head) {
  try {
    build(layers, logit_scale);
  } catch (...) {
    release_all();
    throw;
  }
}

void DorySession::build(const xtg_dory_layer* layers, const float* logit_scale) {
  const xtg_dory_config& c = c_;
  const int n_layers = c.n_in + c.n_rec + c.n_out;
  XTG_CHECK(n_layers > 0 && c.loops >= 1, "dory: %d sublayers, %d loops", n_layers, c.loops);
  XTG_CHECK(c.heads % c.kv_heads == 0 && c.head_dim % 2 == 0, "dory: unsupported attention shape");
  XTG_CHECK(c.kv_mode == XTG_KV_PER_LOOP || c.kv_mode == XTG_KV_LAST_LOOP, "dory: kv_mode %d (per_loop | last_loop)",
            c.kv_mode);
  const int H = c.hidden, Q = c.heads * c.head_dim, KV = c.kv_heads * c.head_dim, F = c.ffn;
  layers_.resize(size_t(n_layers));
  for (int l = 0; l < n_layers; ++l) {
    Layer& L = layers_[size_t(l)];
    L.w = layers[l];
    L.recurrent = l >= c.n_in && l < c.n_in + c.n_rec;
    L.lr = upload(L.w.lr, size_t(H));
    // the fused one-token path's operand of the next projection in the slerp's linear form: a = (1 - lr) x with
    // |x_i| <= 1 (a unit row), b = lr o with |o_i| <= |W_i| |u| <= sqrt(K) max |w| (u, the projection's operand, a
    // unit row); a little margin for rounding
    {
      const xtg_nvfp4& wo = L.w.kind == XTG_DORY_MLP ? L.w.down : L.w.o;
      double la = 0.0, lb = 0.0;
      for (int i = 0; i < H; ++i) {
        la = std::max(la, std::fabs(1.0 - double(L.w.lr[i])));
        lb = std::max(lb, std::fabs(double(L.w.lr[i])));
      }
      L.lin_a = operand_factor(la * 1.01);
      L.lin_b = operand_factor(lb * std::sqrt(double(wo.k)) * max_abs_weight(wo) * 1.01);
    }
    if (L.w.kind == XTG_DORY_MLP) {
      for (const xtg_nvfp4* w : {&L.w.gate, &L.w.up, &L.w.down}) prepare(*w);
      XTG_CHECK(L.w.gate.n_out == F && L.w.up.n_out == F && L.w.gate.k == H && L.w.down.k == F && L.w.down.n_out == H,
                "dory: MLP sublayer %d has the wrong shapes", l);
      L.sg = upload(L.w.sg, size_t(F));
      L.su = upload(L.w.su, size_t(F));
    } else {
      XTG_CHECK(L.w.kind == XTG_DORY_SLIDING || L.w.kind == XTG_DORY_FULL, "dory: sublayer %d kind %d", l, L.w.kind);
      for (const xtg_nvfp4* w : {&L.w.q, &L.w.k, &L.w.v, &L.w.g, &L.w.o}) prepare(*w);
      XTG_CHECK(L.w.q.n_out == Q && L.w.k.n_out == KV && L.w.v.n_out == KV && L.w.g.n_out == Q && L.w.q.k == H &&
                    L.w.o.k == Q && L.w.o.n_out == H,
                "dory: attention sublayer %d has the wrong shapes", l);
      L.qscale = upload(L.w.qscale, size_t(Q));
      L.gscale = upload(L.w.gscale, size_t(Q));
      L.attn = n_attn_++;
      // the session's caches (dory.cpp:436-447): per_loop, one per loop for a recurrent sublayer; last_loop, one
      const int inst = L.recurrent && c.kv_mode == XTG_KV_PER_LOOP ? c.loops : 1;
      for (int i = 0; i < c.loops; ++i)
        caches_.push_back(i < inst ? b_.kv_create(c.kv_heads, c.head_dim, c.context,
                                                   L.w.kind == XTG_DORY_SLIDING ? c.ring_slots : 0, c.kv_dtype)
                                   : nullptr);
      // the RoPE rows of every position the session can reach, made before any capture
      b_.rope_table(L.w.kind == XTG_DORY_SLIDING ? c.theta_sliding : c.theta_full, c.head_dim, c.context);
    }
  }
  if (head_.codes) {   // else a BF16 head comes with set_head_bf16
    prepare(head_);
    XTG_CHECK(head_.k == H && head_.n_out == c.vocab, "dory: LM head %dx%d for hidden %d, vocab %d", head_.n_out,
              head_.k, H, c.vocab);
  }
  logit_scale_ = upload(logit_scale, size_t(c.vocab));
  auto scratch = [&](size_t floats) {
    float* p = static_cast<float*>(b_.alloc(floats * sizeof(float)));
    owned_.push_back(p);
    return p;
  };
  const size_t R = kChunkRows;
  x_ = scratch(R * H);
  x2_ = scratch(R * H);
  part_s_ = scratch(size_t(kMaxFusedGroups) * 5);
  part_h_ = scratch(size_t(kMaxFusedGroups));
  part_a_ = scratch(size_t(c.heads));
  att_ = scratch(size_t(c.heads) * size_t(c.head_dim));
  // XTG_DECODE_UNFUSED=1 runs one-token steps on the separate norm launches (the prefill path's), for comparison;
  // so do models whose shapes some fused projection is not made for
  fused_ = !std::getenv("XTG_DECODE_UNFUSED") && fused_unsupported().empty();
  // XTG_VERIFY_WHOLE_K=1: steps of several rows keep the whole K in their projections (for comparison)
  ksplit_ = !std::getenv("XTG_VERIFY_WHOLE_K");
  input_ = scratch(R * H);
  state_ = scratch(R * H);
  proj_ = scratch(R * size_t(2 * Q + 2 * KV));
  gu_ = scratch(R * 2 * size_t(F));
  o_ = scratch(R * H);
  for (auto* op : {&op_h_, &op_q_, &op_f_, &op_last_}) {
    const int k = op == &op_q_ ? Q : op == &op_f_ ? F : H;
    *op = b_.alloc(Backend::op_bytes(k) * (op == &op_last_ ? 1 : size_t(kChunkRows / 8)));
    owned_.push_back(*op);
  }
  // the slerp's linear-form operand (K = hidden): its entries past hidden and past the four live columns are never
  // written and stay zero
  op_lin_ = b_.alloc(xop_bytes(H));
  owned_.push_back(op_lin_);
  {
    const std::vector<uint8_t> zeros(xop_bytes(H), 0);
    b_.write(op_lin_, 0, zeros.data(), zeros.size());
  }
}

std::string DorySession::fused_unsupported() {
  // every launch sublayer_decode and head can make, with the most records any producer of a slerp leaves (the o and
  // down projections), checked before the first step rather than thrown on it
  auto desc = [&](const xtg_nvfp4* ws, int nw, int in, int out, int groups) {
    FusedGemv f;
    f.c.nw = nw;
    for (int i = 0; i < nw; ++i) f.c.w[i] = &b_.prepare(ws[i]);
    f.c.m = 1;
    f.c.k = ws[0].k;
    f.in = in;
    f.out = out;
    f.in_groups = groups;
    return f;
  };
  int slerp_groups = 1;
  for (const Layer& L : layers_) {
    const bool mlp = L.w.kind == XTG_DORY_MLP;
    const FusedGemv p = desc(mlp ? &L.w.down : &L.w.o, 1, kInNorm, kOutSlerp, 1);
    slerp_groups = std::max(slerp_groups, fused_gemv_groups(p));
  }
  std::string why;
  auto check = [&](const FusedGemv& f, const char* what) {
    if (!why.empty()) return;
    const std::string w = fused_gemv_unsupported(f);
    if (!w.empty()) why = strf("%s: %s", what, w.c_str());
  };
  for (const Layer& L : layers_) {
    if (L.w.kind == XTG_DORY_MLP) {
      const xtg_nvfp4 gu[2] = {L.w.gate, L.w.up};
      int groups = 0;
      for (int in : {kInOp, kInSlerp}) {   // the first projection of a step, or one after a slerp
        const FusedGemv f = desc(gu, 2, in, kOutSwiglu, in == kInSlerp ? slerp_groups : 0);
        check(f, "gate/up");
        groups = std::max(groups, fused_gemv_groups(f));
      }
      check(desc(&L.w.down, 1, kInNorm, kOutSlerp, groups), "down");
    } else {
      const xtg_nvfp4 qkvg[4] = {L.w.q, L.w.k, L.w.v, L.w.g};   // after a prepared operand: the plain GEMV
      check(desc(qkvg, 4, kInSlerp, kOutPlain, slerp_groups), "q/k/v/g");
      check(desc(&L.w.o, 1, kInNorm, kOutSlerp, c_.heads), "o");
    }
  }
  if (head_.codes) check(desc(&head_, 1, kInSlerp, kOutPlain, slerp_groups), "head");
  return why;
}

void DorySession::release_all() {
  try {
    for (auto& snap : snaps_)
      for (DevKv* c : snap) b_.kv_destroy(c);
    for (DevKv* c : caches_)
      if (c) b_.kv_destroy(c);
    for (void* p : owned_) b_.release(p);
    for (const void* key : held_) b_.unhold(key);
  } catch (...) {
  }
  caches_.clear();
  snaps_.clear();
  owned_.clear();
  held_.clear();
}

DorySession::~DorySession() { release_all(); }

DevKv* DorySession::cache(int attn, int inst) {
  XTG_CHECK(attn >= 0 && attn < n_attn_ && inst >= 0 && inst < c_.loops, "dory: no cache %d / %d", attn, inst);
  DevKv* c = caches_[size_t(attn) * size_t(c_.loops) + size_t(inst)];
  XTG_CHECK(c, "dory: attention sublayer %d has no loop instance %d", attn, inst);
  return c;
}

void DorySession::snapshot(int slot) {
  XTG_CHECK(slot >= 0 && slot < kMaxSnapshots, "dory: snapshot slot %d (0..%d)", slot, kMaxSnapshots - 1);
  if (size_t(slot) >= snaps_.size()) snaps_.resize(size_t(slot) + 1);
  std::vector<DevKv*>& snap = snaps_[size_t(slot)];
  size_t i = 0;
  for (DevKv* c : caches_) {
    if (!c || !c->ring) continue;
    if (i == snap.size())   // first use of the slot: a ring like this one
      snap.push_back(b_.kv_create(c->kv_heads, c->head_dim, c->slots, int(c->slots), c->fp8 ? XTG_KV_FP8 : XTG_KV_BF16));
    b_.kv_copy(c, snap[i++]);
  }
}

void DorySession::restore(int slot) {
  XTG_CHECK(slot >= 0 && size_t(slot) < snaps_.size() && !snaps_[size_t(slot)].empty(),
            "dory: snapshot slot %d holds nothing", slot);
  const std::vector<DevKv*>& snap = snaps_[size_t(slot)];
  size_t i = 0;
  for (DevKv* c : caches_)
    if (c && c->ring) b_.kv_copy(snap[i++], c);
}

void DorySession::set_head_bf16(const xtg_bf16& head) {
  XTG_CHECK(head.data && head.n_out == c_.vocab && head.k == c_.hidden,
            "dory: BF16 LM head %dx%d for hidden %d, vocab %d", head.n_out, head.k, c_.hidden, c_.vocab);
  const bool fresh = !b_.has_bf16(head.data);
  b_.prepare(head);
  b_.hold(head.data, fresh);
  held_.push_back(head.data);
  if (head_bf16_.data) {   // the head it replaces
    b_.unhold(head_bf16_.data);
    held_.erase(std::find(held_.begin(), held_.end(), static_cast<const void*>(head_bf16_.data)));
  }
  head_bf16_ = head;
}

void DorySession::sublayer(Layer& L, int m, long long pos0, int inst, bool store) {
  // packs/dory/dory.cpp:467-518; x's GEMV operand is in op_h_ on entry and on exit
  const int H = c_.hidden, Q = c_.heads * c_.head_dim, KV = c_.kv_heads * c_.head_dim, F = c_.ffn;
  // steps of 2..8 rows: the gate/up, down and o projections split K in two (GemvCall::ksplit), and the norm launch
  // that reads their outputs adds the halves; prompt chunks (the GEMM) and single rows keep one output set
  const int ks = ksplit_ && m >= 2 ? 2 : 1;
  if (L.w.kind == XTG_DORY_MLP) {
    const xtg_nvfp4 gu[2] = {L.w.gate, L.w.up};
    const int gp = b_.matmul_op(gu, 2, op_h_, m, gu_, 0, nullptr, ks);  // gate rows [m][F], then up rows
    b_.swiglu_norm(gu_, gu_ + size_t(m) * F, L.sg, L.su, m, F, nullptr, op_f_,
                   gp == 2 ? size_t(m) * 2 * F : 0);   // justnorm(silu(g sg) (u su))
    const int dp = b_.matmul_op(&L.w.down, 1, op_f_, m, o_, 0, nullptr, ks);
    b_.slerp_norm(x_, o_, L.lr, m, H, op_h_, dp == 2 ? size_t(m) * H : 0);
    return;
  }
  const xtg_nvfp4 qkvg[4] = {L.w.q, L.w.k, L.w.v, L.w.g};
  b_.matmul_op(qkvg, 4, op_h_, m, proj_, 0);   // q [m][Q] | k [m][KV] | v [m][KV] | g [m][Q]
  float* q = proj_;
  float* k = proj_ + size_t(m) * Q;
  float* v = k + size_t(m) * KV;
  float* g = v + size_t(m) * KV;
  const bool sliding = L.w.kind == XTG_DORY_SLIDING;
  const float scale = 1.f / std::sqrt(float(c_.head_dim));
  b_.attn_step(this->cache(L.attn, inst), m, pos0, c_.heads, sliding ? c_.window : 0, scale,
               sliding ? c_.theta_sliding : c_.theta_full, q, k, v, L.qscale, g, L.gscale, nullptr, op_q_, store);
  const int op = b_.matmul_op(&L.w.o, 1, op_q_, m, o_, 0, nullptr, ks);
  b_.slerp_norm(x_, o_, L.lr, m, H, op_h_, op == 2 ? size_t(m) * H : 0);
}

void DorySession::materialize(int m) {
  if (!pend_) return;
  b_.slerp_norm(x_, o_, pend_lr_, m, c_.hidden, op_h_);
  if (pend_post_ == kPostAddNorm) b_.add_norm(x_, x_, x_, m, c_.hidden, op_h_);
  if (pend_post_ == kPostNorm) b_.add_norm(x_, nullptr, x_, m, c_.hidden, op_h_);
  pend_ = false;
  pend_post_ = kPostNone;
}

void DorySession::sublayer_decode(Layer& L, int m, long long pos0, int inst, bool store) {
  // packs/dory/dory.cpp:467-518 for one token: the slerp closing the previous sublayer is made by this sublayer's
  // first projection, the SwiGLU norm by the down projection, and this sublayer's slerp is left to the next
  const int Q = c_.heads * c_.head_dim, KV = c_.kv_heads * c_.head_dim;
  auto input_side = [&](FusedGemv& f) {
    if (!pend_) return;   // op_h_ holds x's operand
    f.in = kInSlerp;      // op_lin_ holds the slerp's linear-form operand
    f.in_x = x_;
    f.in_o = o_;
    f.in_lr = pend_lr_;
    f.in_part = part_s_;
    f.in_groups = pend_groups_;
    f.in_xout = x2_;
    f.in_ia = 1.f / pend_a_;
    f.in_ib = 1.f / pend_b_;
    f.in_post = pend_post_;
  };
  const void* in_op = pend_ ? op_lin_ : op_h_;
  auto slerp_side = [&](FusedGemv& f) {
    f.out = kOutSlerp;
    f.out_x = x_;
    f.out_lr = L.lr;
    f.out_part = part_s_;
    f.out_op = op_lin_;
    f.out_ea = L.lin_a;
    f.out_eb = L.lin_b;
  };
  auto pending = [&](int groups) {
    pend_groups_ = groups;
    pend_ = true;
    pend_lr_ = L.lr;
    pend_a_ = L.lin_a;
    pend_b_ = L.lin_b;
  };
  auto took_input = [&] {
    if (!pend_) return;
    std::swap(x_, x2_);   // the projection wrote the new residual
    pend_ = false;
    pend_post_ = kPostNone;
  };
  if (L.w.kind == XTG_DORY_MLP) {
    const xtg_nvfp4 gu[2] = {L.w.gate, L.w.up};
    FusedGemv g;
    input_side(g);
    g.out = kOutSwiglu;
    g.out_sg = L.sg;
    g.out_su = L.su;
    g.out_part = part_h_;
    const int groups = b_.matmul_fused(gu, 2, g, in_op, m, gu_);   // h = silu(g sg) (u su) [m][F]
    took_input();
    FusedGemv d;
    d.in = kInNorm;   // justnorm(h) as the operand
    d.in_x = gu_;
    d.in_part = part_h_;
    d.in_groups = groups;
    slerp_side(d);
    pending(b_.matmul_fused(&L.w.down, 1, d, nullptr, m, o_));
    return;
  }
  const xtg_nvfp4 qkvg[4] = {L.w.q, L.w.k, L.w.v, L.w.g};
  FusedGemv p;
  input_side(p);
  b_.matmul_fused(qkvg, 4, p, in_op, m, proj_);   // q [m][Q] | k [m][KV] | v [m][KV] | g [m][Q]
  took_input();
  float* q = proj_;
  float* k = proj_ + size_t(m) * Q;
  float* v = k + size_t(m) * KV;
  float* g = v + size_t(m) * KV;
  const bool sliding = L.w.kind == XTG_DORY_SLIDING;
  const float scale = 1.f / std::sqrt(float(c_.head_dim));
  // the gate's justnorm rides on the o-projection: att_ holds the gated heads, part_a_ their sums of squares
  b_.attn_step(this->cache(L.attn, inst), m, pos0, c_.heads, sliding ? c_.window : 0, scale,
               sliding ? c_.theta_sliding : c_.theta_full, q, k, v, L.qscale, g, L.gscale, att_, nullptr, store,
               part_a_);
  FusedGemv o;
  o.in = kInNorm;
  o.in_x = att_;
  o.in_part = part_a_;
  o.in_groups = c_.heads;
  slerp_side(o);
  pending(b_.matmul_fused(&L.w.o, 1, o, nullptr, m, o_));
}

void DorySession::run_chunk(const float* x, int m, long long pos0, bool keep_pending) {
  // packs/dory/dory.cpp:520-544 from the embedding rows; x's operand is in op_h_ on exit
  XTG_CHECK(m >= 1 && m <= kChunkRows, "dory: %d rows per chunk (1..%d)", m, kChunkRows);
  XTG_CHECK(pos0 >= 0 && pos0 + m <= c_.context, "context full: %lld + %d > %lld tokens", pos0, m,
            (long long)c_.context);
  const int H = c_.hidden;
  const size_t bytes = size_t(m) * H * sizeof(float);
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    b_.prep_x(x, XTG_X_F32, m, H, op_h_, x_);   // the rows' operand, and the rows into x_
  } else {
    b_.copy(x, 0, x_, 0, bytes);
    b_.prep_x(x_, XTG_X_F32, m, H, op_h_);
  }
  const bool fused = fused_ && m == 1;   // several rows take the separate norm launches
  pend_ = false;
  auto run = [&](Layer& L, int inst, bool store) {
    if (fused)
      sublayer_decode(L, m, pos0, inst, store);
    else
      sublayer(L, m, pos0, inst, store);
  };
  size_t l = 0;
  for (; l < size_t(c_.n_in); ++l) run(layers_[l], 0, true);
  // One loop and a slerp pending: the loop's entry and exit norms ride on the next projection (in_post), since
  // neither state nor input is read again. Otherwise they run on the materialized residual.
  const bool fold = c_.loops == 1 && c_.n_rec > 0;
  if (fold && pend_) {
    pend_post_ = kPostAddNorm;
  } else {
    materialize(m);
    // the loops start from state = input = x: the first entry is justnorm(x + x) read in place, and input is kept
    // only for later entries; the last exit writes x in place (x = state = justnorm(x))
    if (c_.loops > 1) b_.copy(x_, 0, input_, 0, bytes);
    b_.add_norm(x_, x_, x_, m, H, op_h_);   // x = justnorm(state + input), state = input = x
  }
  for (int i = 0; i < c_.loops; ++i) {
    const bool last = i == c_.loops - 1;
    if (i > 0) b_.add_norm(state_, input_, x_, m, H, op_h_);   // x = justnorm(state + input)
    // last_loop: every loop attends to the chunk's own keys, the cache keeps the last loop's (dory.cpp:534-537)
    const bool per_loop = c_.kv_mode == XTG_KV_PER_LOOP;
    for (size_t r = size_t(c_.n_in); r < size_t(c_.n_in + c_.n_rec); ++r)
      run(layers_[r], per_loop ? i : 0, per_loop || last);
    if (fold && pend_ && pend_post_ == kPostNone) {
      pend_post_ = kPostNorm;   // x = state = justnorm(x)
    } else {
      materialize(m);
      b_.add_norm(x_, nullptr, last ? x_ : state_, m, H, last ? op_h_ : nullptr);   // state = justnorm(x)
    }
  }
  for (l = size_t(c_.n_in + c_.n_rec); l < layers_.size(); ++l) run(layers_[l], 0, true);
  if (!keep_pending) materialize(m);
}

void DorySession::head(int r0, int rows, float* logits) {
  // the head times logit_scale (dory.cpp:566-575) for chunk rows r0 .. r0 + rows - 1 into logits [rows][vocab]
  const int H = c_.hidden;
  const float* x = x_ + size_t(r0) * H;
  if (head_bf16_.data) {   // from the FP32 rows: the BF16 GEMV makes its own three-term operand, 8 rows a call
    for (int r = 0; r < rows; r += 8)
      b_.matmul_bf16_dev(head_bf16_, x + size_t(r) * H, XTG_X_F32, std::min(8, rows - r), logits,
                         size_t(r) * size_t(c_.vocab), logit_scale_);
    return;
  }
  XTG_CHECK(head_.codes, "dory: no LM head (pass an NVFP4 head to create or set a BF16 one)");
  if (pend_) {   // one row whose last slerp is pending: it rides on the head's projection, which writes x too
    XTG_CHECK(r0 == 0 && rows == 1, "dory: a pending slerp for head rows %d .. %d", r0, r0 + rows - 1);
    FusedGemv f;
    f.in = kInSlerp;
    f.in_x = x_;
    f.in_o = o_;
    f.in_lr = pend_lr_;
    f.in_part = part_s_;
    f.in_groups = pend_groups_;
    f.in_xout = x2_;
    f.in_ia = 1.f / pend_a_;
    f.in_ib = 1.f / pend_b_;
    f.in_post = pend_post_;
    f.c.col_scale[0] = logit_scale_;
    b_.matmul_fused(&head_, 1, f, op_lin_, 1, logits);
    std::swap(x_, x2_);
    pend_ = false;
    pend_post_ = kPostNone;
    return;
  }
  const void* op = op_h_;   // the chunk's operand when the rows are all of it, else the rows' own
  if (r0 != 0) {
    XTG_CHECK(rows == 1, "dory: head rows %d .. %d of a chunk", r0, r0 + rows - 1);
    b_.prep_x(x, XTG_X_F32, 1, H, op_last_);
    op = op_last_;
  }
  b_.matmul_op(&head_, 1, op, rows, logits, 0, logit_scale_);
}

void DorySession::forward(const float* x, int m, long long pos0, float* logits) {
  // one chunk, then the head over all its rows (dory.cpp:566-576 with Logits::All)
  run_chunk(x, m, pos0, m == 1 && !head_bf16_.data && head_.codes);
  head(0, m, logits);
}

void DorySession::prefill(const float* x, int n, long long pos0, int want, float* logits) {
  // DorySession::forward (dory.cpp:554-578): chunks of up to 512 rows; logits for every row (ALL, [n][vocab]),
  // the last row (LAST, [vocab]) or none
  XTG_CHECK(n >= 1, "dory: %d rows", n);
  XTG_CHECK(want == XTG_LOGITS_NONE || want == XTG_LOGITS_LAST || want == XTG_LOGITS_ALL, "dory: logits mode %d",
            want);
  XTG_CHECK(want == XTG_LOGITS_NONE || logits, "dory: NULL logits");
  XTG_CHECK(pos0 >= 0 && pos0 + n <= c_.context, "context full: %lld + %d > %lld tokens", pos0, n,
            (long long)c_.context);
  for (int off = 0; off < n; off += kChunkRows) {
    const int m = std::min(kChunkRows, n - off);
    run_chunk(x + size_t(off) * size_t(c_.hidden), m, pos0 + off);
    if (want == XTG_LOGITS_ALL) head(0, m, logits + size_t(off) * size_t(c_.vocab));
    else if (want == XTG_LOGITS_LAST && off + m == n) head(m - 1, 1, logits);
  }
}

}  // namespace xtg::hip
