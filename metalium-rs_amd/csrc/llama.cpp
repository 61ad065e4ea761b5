// The Llama / SmolLM2 decoder harness over the engine.
//
// Reference: crates/tt-models/src/llama.rs -- the config (40-71), a layer's
// pre-norm attention and SwiGLU MLP (140-520), the tied head on the last
// position (1030-1090), greedy generation (1136-1178); the KV cache written
// by slice_assign (415-435) and grouped-query attention (437-455);
// crates/tt-models/src/rope.rs:1-140 for the rotary tables.
//
// Layout on the device.  Activations are F32 [batch * t, hidden], row
// (sequence, position).  Projection weights are BF16 stored [out, in], so
// every product reads its weight k-contiguous: the decode GEMV streams each
// weight row once; prefill runs the MFMA kernels.  Each layer's q|k|v and
// gate|up weights are one matrix each (the reference's `Llama::fused`,
// llama.rs:655-672): prefill multiplies by row blocks of them, and a decode
// step of at most 32 sequences runs six fused launches a layer -- RMSNorm +
// q|k|v + RoPE + cache write, attention (two), o + residual, RMSNorm +
// gate|up + SiLU-mul, down + residual.  The KV cache of a layer is
// [batch * kv_heads * max_ctx, head_dim], item (sequence, kv head), F32 under
// the reference numeric contract and BF16 under the performance one (which
// also rounds a prefill product's activation operand to BF16), so the
// attention of a query group is one product over a block of the cache:
// queries regrouped to [batch * kv_heads, t * group, head_dim] (row
// t * group + g) multiply the first ctx rows of their cache item.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/miburn_models.h"
#include "burn.hpp"

namespace {

thread_local std::string g_model_error;

using burn::Tensor;

struct Layer {
  Tensor attn_norm, wqkv, wo, mlp_norm, wgu, wdown;  // wqkv = [wq; wk; wv], wgu = [gate; up]
  // wgu's rows interleaved in 32-row groups (gate 0..31, up 0..31, gate
  // 32..63, ...) for mi_linear_swiglu_parts (intermediate a multiple of 128;
  // weights do not change after creation).
  Tensor wgu_pairs;
  // Under the performance contract the four projection weights are BFP8
  // (the reference's Numerics::Performance weight plan, crates/tt-models/src/
  // quant.rs:154-175: every matrix but the embedding table).  A decode step
  // reads these as stored (1 + 1/16 bytes a weight); the BF16 tensors above
  // then hold the same values decoded (exact), for the prefill's matrix-core
  // products, whose time is arithmetic, not weight bytes.
  Tensor q_wqkv, q_wo, q_wgu, q_wdown;
  // The four projection weights again in the matrix cores' operand order
  // (mi_tile; gate|up interleaved as wgu_pairs), for the products of a prompt
  // of up to kTilesMaxRows rows (mi_linear's short-row path).
  Tensor t_wqkv, t_wo, t_wgu_pairs, t_wdown;
  Tensor cache_k, cache_v;
};

}  // namespace

// A decode step captured as a trace (mi_llama_generate_traced): its span and
// the buffer its replays leave the next token ids in.
struct StepTrace {
  uint64_t id = 0;
  Tensor next;  // [batch, 1] I32, allocated by the capture
};

// A prompt's prefill from position 0 captured as a trace, per (batch,
// length): its token ids input and the buffer its replays leave the first new
// ids in.  id 0: the prefill could not be captured (its path uploads, as the
// composition's causal mask does) and runs eagerly.
struct PromptTrace {
  uint64_t id = 0;
  Tensor ids, next;  // [batch * t] and [batch, 1] I32
};

struct mi_llama {
  mi_ctx *ctx;
  mi_llama_config cfg;
  Tensor embed, final_norm;
  std::vector<Layer> layers;
  Tensor rope_cos, rope_sin;  // [max_ctx, head_dim]
  int64_t len = 0;            // positions in the cache
  int64_t cache_batch = 0;    // sequences the cache holds
  // Traced decode steps over the current caches, by span; their inputs: the
  // token ids [batch, 1] and the position [1, 1] (I32).
  std::map<int64_t, StepTrace> traces;
  Tensor step_ids, step_pos;
  // [batch, max_ctx] I32: the token each chained step chose, at the
  // position it goes to (mi_decode_advance), read back once a generation.
  Tensor step_log;
  std::map<std::pair<int64_t, int64_t>, PromptTrace> prompt_traces;
};

namespace {

int fail_model(const std::exception &e) {
  g_model_error = e.what();
  if (auto *be = dynamic_cast<const burn::Error *>(&e)) return be->status;
  return MI_E_ARG;
}

Tensor weight(mi_ctx *ctx, int64_t rows, int64_t cols, float stdv, uint64_t base) {
  Tensor w = burn::random(ctx, {rows, cols}, MI_DRAW_NORMAL, 0.0f, stdv, base);
  return burn::float_cast(w, MI_BF16);
}

// Largest number of new positions per sequence that take the fused attention.
constexpr int64_t kFusedAttentionMaxT = 16;
// Long prompts of a few sequences take the fused kernel too: a 512-token
// prefill at batch 1 in 4.0-4.2 ms against 5.3 through the composition
// (scores, masked softmax, P V and the regroup never touch HBM); at batch 32
// the composition's matrix-core products win (37 against 43.5 ms).
constexpr int64_t kFusedAttentionLongMaxBatch = 4;
// New positions from which mi_attention_rows runs 64-wide heads on the
// matrix cores (its flash kernel, keys split into ranges on small grids).
constexpr int64_t kFlashMinT = 64;
// Largest batch whose decode step takes the fused projections, and whose
// head is one fused norm + projection launch (mi_norm_matvec: the GEMV up to 6
// rows, the matrix-core form above; beyond kFusedHeadMaxBatch the head is a
// plain product).  Under the reference contract the fused head serves every
// decode batch (batch-32 SmolLM2 decode 1.645 -> 1.621 ms a step: the plain
// F32 x BF16 product of 32 rows ran on the F32 matrix cores); the
// performance contract's BF16 product stays ahead above 8 (1.577 against
// 1.587).
constexpr int64_t kDecodeMaxBatch = 32;
constexpr int64_t kFusedHeadMaxBatch = 8;
// A decode step's attention plans its key chunks for its span: the attended
// positions rounded up to a multiple of kSpanStep (at most max_ctx).  Every
// step of one span runs the same launches, so a step captured once replays
// at each of its positions, and an eager step computes the same bits.
constexpr int64_t kSpanStep = 64;
// Prompts of up to this many rows (sequences x positions, a multiple of 32)
// run their projections against the tiled weights: one block a 32 x 32 (or
// 32 x 64) output tile with k split over its waves, the activations handed
// over in tiles by the norms and the SwiGLU.
constexpr int64_t kTilesMaxRows = 2048;

int64_t decode_span(const mi_llama *m, int64_t ctxlen) {
  return std::min<int64_t>(m->cfg.max_ctx, (ctxlen + kSpanStep - 1) / kSpanStep * kSpanStep);
}

// Whether a single-position step of `batch` sequences takes the fused decode
// launches (and so can be traced).
bool decode_fused(const mi_llama *m, int64_t batch) {
  const mi_llama_config &c = m->cfg;
  const int64_t D = c.head_dim, G = c.heads / c.kv_heads;
  return batch <= kDecodeMaxBatch && (D == 16 || D == 32 || D == 64 || D == 128) && G <= 8 && c.hidden % 8 == 0 &&
         c.intermediate % 8 == 0;
}

// The layers of a decode step on the hidden rows x [batch, hidden]: the new
// position pos0 (immediate) or held on the device in `pos`, the attention
// planned for `span` positions.  Four launches a layer for one sequence (q|k|v
// and the attention's chunks in one, their combine in the o projection's),
// five up to 6 sequences, six above.
Tensor decode_layers(mi_llama *m, Tensor x, int64_t batch, const Tensor *pos, int64_t pos0, int64_t span) {
  const mi_llama_config &c = m->cfg;
  const int64_t H = c.heads, KVH = c.kv_heads, D = c.head_dim;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));
  for (Layer &L : m->layers) {
    const bool q = L.q_wqkv.defined();  // BFP8 weights
    x = burn::norm_qkv_attention_o(x, L.attn_norm, c.eps, q ? L.q_wqkv : L.wqkv, m->rope_cos, m->rope_sin, H, KVH,
                                   pos, pos0, span, L.cache_k, L.cache_v, scale, q ? L.q_wo : L.wo);
    Tensor h = burn::norm_matvec(x, &L.mlp_norm, c.eps, q ? L.q_wgu : L.wgu, nullptr, true);
    x = burn::norm_matvec(h, nullptr, 0.0f, q ? L.q_wdown : L.wdown, &x, false);
  }
  return x;
}

Tensor ones(mi_ctx *ctx, int64_t n) { return burn::fill(ctx, {1, n}, MI_F32, 0x3f800000u); }

// Whether a prefill product of `rows` F32 activation rows against a BF16
// weight [n, k] takes the activations' BF16 parts from their producer
// (RMSNorm, the SiLU-mul write MI_BF16_PARTS) into mi_linear_parts: in the
// fast matmul mode, from 4096 rows in 128-row tiles.  Where the library
// would split the activations itself into parts for its direct kernel
// (rows in 256-row tiles over at least 128 tiles of 256 x 256) the result is
// the same with no split pass between; from 4096 rows the direct kernel on
// parts also beats the split kernel (SmolLM2 shapes at 4096 rows, us: q|k|v
// 33.7 -> 17.8, gate|up 51.2 -> 44.4, down 39.8 -> 38.1; at 2048 rows and
// below the split kernel stays ahead).
static bool parts_pay(mi_ctx *ctx, int64_t rows, int64_t k, int64_t n) {
  int mode = MI_MATMUL_ACCURATE;
  if (mi_get_matmul_mode(ctx, &mode) != MI_OK || mode != MI_MATMUL_FAST) return false;
  return rows >= 4096 && rows % 128 == 0 && k % 32 == 0 && n % 16 == 0;
}

// The forward of `t` positions per sequence at cache length m->len; returns
// the hidden states [batch * t, hidden] before the final norm.
// The hidden rows of token ids already on the device ([batch * t] I32, rows
// (sequence, position)).
// A prefill's attention over q from the q|k|v tail (rows (sequence,
// position, head) for the fused kernel, else regrouped per kv head): the
// output rows (sequence, position) of heads x head_dim.
Tensor attention_of(mi_llama *m, Layer &L, const Tensor &q, int64_t batch, int64_t t, int64_t pos0, int64_t ctxlen,
                    bool fused, const Tensor &mask, float scale) {
  const mi_llama_config &c = m->cfg;
  const int64_t H = c.heads, KVH = c.kv_heads, D = c.head_dim, G = H / KVH, maxc = c.max_ctx, rows = batch * t;
  if (fused) return burn::attention_rows(q.reshape({rows, H * D}), L.cache_k, L.cache_v, batch, t, H, KVH, pos0, scale);
  // [batch * KVH * t * G, D], rows (p, g) of each (sequence, kv head)
  Tensor scores = burn::matmul_blocks(q, false, L.cache_k, true, batch * KVH, t * G, D, ctxlen, 0, t * G * D, 0,
                                      maxc * D);
  Tensor p = burn::softmax_rows(scores, mask.defined() ? &mask : nullptr, scale, false);
  Tensor o = burn::matmul_blocks(p, false, L.cache_v, false, batch * KVH, t * G, ctxlen, D, 0, t * G * ctxlen, 0,
                                 maxc * D);
  // Back to rows (sequence, position), heads in order h = j * G + g.
  const int64_t dims[4] = {batch, t, KVH, G * D};
  const int64_t st[4] = {KVH * t * G * D, G * D, t * G * D, 1};
  return burn::copy4(o, dims, 0, st).reshape({rows, H * D});
}

Tensor forward_ids(mi_llama *m, const Tensor &idx, int64_t batch, int64_t t) {
  mi_ctx *ctx = m->ctx;
  const mi_llama_config &c = m->cfg;
  const int64_t H = c.heads, KVH = c.kv_heads, D = c.head_dim, G = H / KVH;
  const int64_t pos0 = m->len, ctxlen = pos0 + t;
  const int64_t rows = batch * t;

  // The element type of a prefill product's activation operand.
  const int act = c.numerics == MI_NUMERICS_PERFORMANCE ? MI_BF16 : MI_F32;
  Tensor x = burn::select_rows_as(m->embed, idx, MI_F32);  // [rows, hidden], the BF16 rows widened
  x = x.reshape({rows, c.hidden});

  // A few new positions (decode) take the fused attention kernel, and so does
  // a long prompt with 64-wide heads (the matrix-core flash kernel behind
  // mi_attention_rows) or of a few sequences; other long prompts take the
  // product composition.
  const bool fused = (t <= kFusedAttentionMaxT || batch <= kFusedAttentionLongMaxBatch ||
                      (D == 64 && t >= kFlashMinT)) &&
                     (D == 16 || D == 32 || D == 64 || D == 128) && G <= 8;
  // The composition's causal mask for t > 1, rows (position, group) of one
  // item: row p * G + g attends to cache columns <= pos0 + p.
  Tensor mask;
  if (t > 1 && !fused) {
    std::vector<uint32_t> mk(static_cast<size_t>(t * G * ctxlen));
    for (int64_t p = 0; p < t; ++p)
      for (int64_t g = 0; g < G; ++g)
        for (int64_t j = 0; j < ctxlen; ++j) mk[(p * G + g) * ctxlen + j] = j > pos0 + p ? 1u : 0u;
    mask = burn::bool_from_data(ctx, mk.data(), {t * G, ctxlen});
  }
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));

  if (t == 1 && decode_fused(m, batch)) {
    x = decode_layers(m, x, batch, nullptr, pos0, decode_span(m, ctxlen));
    m->len = ctxlen;
    return x;
  }
  // Under the reference contract, the products the fast mode would split
  // take their activations' parts from the producers.
  const int64_t nqkv = (H + 2 * KVH) * D;
  const bool parts_qkv = act == MI_F32 && parts_pay(ctx, rows, c.hidden, nqkv);
  const bool parts_gu = act == MI_F32 && parts_pay(ctx, rows, c.hidden, 2 * c.intermediate);
  const bool parts_down = act == MI_F32 && parts_pay(ctx, rows, c.intermediate, c.hidden);
  const bool parts_o = act == MI_F32 && parts_pay(ctx, rows, H * D, c.hidden);
  // A layer's attention norm comes with the previous layer's down product
  // (mi_linear_add_rms_norm: where that product splits over k, a short
  // prompt's, its reduce forms the norm; bit for bit the two calls).
  Tensor xn_next;
  // A short prompt's products against the tiled weights, their activations in
  // tiles: the F32 values' parts under the reference contract, BF16 values
  // under the performance one (the attention output goes in as rows).
  int mode = MI_MATMUL_FAST;
  (void)mi_get_matmul_mode(ctx, &mode);
  const bool tiles = !m->layers.empty() && m->layers[0].t_wqkv.defined() && rows % 32 == 0 &&
                     rows <= kTilesMaxRows && (act == MI_BF16 || mode == MI_MATMUL_FAST);
  if (tiles) {
    const int tform = act == MI_F32 ? MI_TILES_PARTS : MI_TILES_BF16;
    for (size_t li = 0; li < m->layers.size(); ++li) {
      Layer &L = m->layers[li];
      Tensor xn = xn_next.defined() ? xn_next : burn::rms_norm(x, L.attn_norm, c.eps, tform);
      xn_next = Tensor();
      Tensor q = burn::linear_qkv_rope_cache(xn, false, L.t_wqkv, m->rope_cos, m->rope_sin, t, H, KVH, pos0, L.cache_k,
                                             L.cache_v, !fused);
      // The attention hands its result to the o projection in tiles (the
      // matrix-core kernel stores them itself).
      Tensor oh = fused ? burn::attention_rows_as(q.reshape({rows, H * D}), L.cache_k, L.cache_v, batch, t, H, KVH, pos0,
                                                  scale, tform)
                        : burn::tile(attention_of(m, L, q, batch, t, pos0, ctxlen, fused, mask, scale), tform);
      Tensor hn;
      std::tie(x, hn) = burn::linear_add_rms_norm(oh, L.t_wo, true, nullptr, &x, L.mlp_norm, c.eps, tform);
      Tensor h = burn::linear_swiglu(hn, L.t_wgu_pairs, tform);
      if (li + 1 < m->layers.size())
        std::tie(x, xn_next) = burn::linear_add_rms_norm(h, L.t_wdown, true, nullptr, &x, m->layers[li + 1].attn_norm,
                                                         c.eps, tform);
      else
        x = burn::linear(h, L.t_wdown, true, nullptr, &x);
    }
    m->len = ctxlen;
    return x;
  }
  for (size_t li = 0; li < m->layers.size(); ++li) {
    Layer &L = m->layers[li];
    Tensor xn = xn_next.defined() ? xn_next : burn::rms_norm(x, L.attn_norm, c.eps, parts_qkv ? MI_BF16_PARTS : act);
    xn_next = Tensor();
    // One product against the fused q|k|v weight, then RoPE on q and k, k and
    // v appended to the caches at positions pos0.. of each (sequence, kv head)
    // item, and q laid out for the attention, in one launch: rows (sequence,
    // position, head) for the fused kernel, else regrouped per kv head, rows
    // (sequence, kv head, position, g).
    // From 4096 rows with 64-wide heads the product's epilogue runs that tail
    // itself (mi_linear_qkv_rope_cache: no F32 q|k|v rows between them), from
    // BF16 activations or the F32 activations' parts (batch 32, from the
    // parts: 54 us a layer against 49 + 28 for the product then the tail
    // kernel; from BF16 activations 35 us).
    Tensor q;
    if (D == 64 && rows >= 4096 && rows % 128 == 0 && c.hidden % 32 == 0 && (act == MI_BF16 || parts_qkv)) {
      q = burn::linear_qkv_rope_cache(xn, parts_qkv, L.wqkv, m->rope_cos, m->rope_sin, t, H, KVH, pos0, L.cache_k,
                                      L.cache_v, !fused);
    } else {
      Tensor qkv = parts_qkv ? burn::linear_parts(xn, L.wqkv, true, nullptr, nullptr)
                             : burn::float_matmul(xn, false, L.wqkv, true);
      q = burn::qkv_rope_cache(qkv, m->rope_cos, m->rope_sin, t, H, KVH, pos0, L.cache_k, L.cache_v, !fused);
    }
    // x + oh wo^T (the add in the product's epilogue), and its MLP norm.
    Tensor hn;
    if (parts_o) {
      // The attention's result as parts, stored by the attention kernels
      // (no split pass before the o product).
      Tensor ohp = fused ? burn::attention_rows_as(q.reshape({rows, H * D}), L.cache_k, L.cache_v, batch, t, H, KVH,
                                                   pos0, scale, MI_BF16_PARTS)
                         : burn::parts(attention_of(m, L, q, batch, t, pos0, ctxlen, fused, mask, scale));
      x = burn::linear_parts(ohp, L.wo, true, nullptr, &x);
      hn = burn::rms_norm(x, L.mlp_norm, c.eps, parts_gu ? MI_BF16_PARTS : act);
    } else {
      // BF16 activations: the attention kernels store the result as BF16.
      Tensor oh;
      if (fused && act == MI_BF16) {
        oh = burn::attention_rows_as(q.reshape({rows, H * D}), L.cache_k, L.cache_v, batch, t, H, KVH, pos0, scale,
                                     MI_BF16);
      } else {
        oh = attention_of(m, L, q, batch, t, pos0, ctxlen, fused, mask, scale);
        if (act != MI_F32) oh = burn::float_cast(oh, act);
      }
      std::tie(x, hn) = burn::linear_add_rms_norm(oh, L.wo, true, nullptr, &x, L.mlp_norm, c.eps,
                                                  parts_gu ? MI_BF16_PARTS : act);
    }
    // One product against the fused gate|up weight, silu(gate) * up of its halves.
    // With parts for both the gate|up and the down product, one launch forms
    // silu(gate) * up's parts from the interleaved weight (no F32 [rows,
    // 2 inter] product in between).
    Tensor h;
    if (parts_gu && parts_down && L.wgu_pairs.defined()) {
      h = burn::linear_swiglu_parts(hn, L.wgu_pairs);
    } else if (act == MI_BF16 && L.wgu_pairs.defined() && rows >= 4096 && rows % 128 == 0) {
      // The performance contract's BF16 activations: the same launch, its
      // result rounded to BF16 for the down product (batch-32 512-token
      // prefill 12.9 -> 12.1 ms; at 512 rows the product then the SiLU-mul
      // stays ahead, 2.35 against 2.50 ms for the prefill).
      h = burn::linear_swiglu(hn, L.wgu_pairs, MI_BF16);
    } else {
      Tensor gu = parts_gu ? burn::linear_parts(hn, L.wgu, true, nullptr, nullptr)
                           : burn::float_matmul(hn, false, L.wgu, true);
      h = burn::silu_mul_halves(gu, parts_down ? MI_BF16_PARTS : act);
    }
    if (parts_down) {
      x = burn::linear_parts(h, L.wdown, true, nullptr, &x);
    } else if (li + 1 < m->layers.size()) {
      std::tie(x, xn_next) = burn::linear_add_rms_norm(h, L.wdown, true, nullptr, &x, m->layers[li + 1].attn_norm, c.eps,
                                                       parts_qkv ? MI_BF16_PARTS : act);
    } else {
      x = burn::linear(h, L.wdown, true, nullptr, &x);
    }
  }
  m->len = ctxlen;
  return x;
}

Tensor forward_hidden(mi_llama *m, const int32_t *ids, int64_t batch, int64_t t) {
  return forward_ids(m, burn::int_from_data(m->ctx, ids, {batch * t}), batch, t);
}

// The final norm and the tied head over the last position of each sequence:
// [batch, vocab].  One position per sequence (up to kFusedHeadMaxBatch
// sequences, or kDecodeMaxBatch under the reference contract): one fused
// norm + projection launch over the embedding table.
Tensor head_last(mi_llama *m, const Tensor &hidden, int64_t batch, int64_t t) {
  const mi_llama_config &c = m->cfg;
  const int64_t fused_max = c.numerics == MI_NUMERICS_PERFORMANCE ? kFusedHeadMaxBatch : kDecodeMaxBatch;
  if (t == 1 && batch <= fused_max && c.hidden % 8 == 0)
    return burn::norm_matvec(hidden, &m->final_norm, c.eps, m->embed, nullptr, false);
  const int64_t dims[4] = {1, 1, batch, c.hidden};
  const int64_t st[4] = {0, 0, t * c.hidden, 1};
  Tensor last = burn::copy4(hidden, dims, (t - 1) * c.hidden, st);
  const int act = c.numerics == MI_NUMERICS_PERFORMANCE ? MI_BF16 : MI_F32;
  return burn::float_matmul(burn::rms_norm(last, m->final_norm, c.eps, act), false, m->embed, true);
}

// The greedy pick of each sequence's last position: [batch, 1] I32 (the
// reference's generation loop, crates/tt-models/src/generate.rs:176-183).
// A decode step's head and pick are one call (mi_norm_matvec_argmax).
Tensor greedy_last(mi_llama *m, const Tensor &hidden, int64_t batch, int64_t t) {
  const mi_llama_config &c = m->cfg;
  const int64_t fused_max = c.numerics == MI_NUMERICS_PERFORMANCE ? kFusedHeadMaxBatch : kDecodeMaxBatch;
  if (t == 1 && batch <= fused_max && c.hidden % 8 == 0)
    return burn::norm_matvec_argmax(hidden, m->final_norm, c.eps, m->embed);
  return burn::argmax_rows(head_last(m, hidden, batch, t));
}

// Every position's logits: [batch * t, vocab].
Tensor head_all(mi_llama *m, const Tensor &hidden) {
  const int act = m->cfg.numerics == MI_NUMERICS_PERFORMANCE ? MI_BF16 : MI_F32;
  return burn::float_matmul(burn::rms_norm(hidden, m->final_norm, m->cfg.eps, act), false, m->embed, true);
}

// Release every captured decode step (they read the current caches).
void drop_traces(mi_llama *m) {
  for (auto &kv : m->traces) (void)mi_trace_release(m->ctx, kv.second.id);
  m->traces.clear();
  for (auto &kv : m->prompt_traces)
    if (kv.second.id) (void)mi_trace_release(m->ctx, kv.second.id);
  m->prompt_traces.clear();
}

void ensure_cache(mi_llama *m, int64_t batch) {
  if (m->len == 0 && m->cache_batch != batch) {
    drop_traces(m);
    const mi_llama_config &c = m->cfg;
    const int kv = c.numerics == MI_NUMERICS_PERFORMANCE ? MI_BF16 : MI_F32;
    for (Layer &L : m->layers) {
      // The old caches go before the new ones are made, so their memory is reused.
      L.cache_k = Tensor();
      L.cache_v = Tensor();
      L.cache_k = burn::fill(m->ctx, {batch * c.kv_heads * c.max_ctx, c.head_dim}, kv, 0);
      L.cache_v = burn::fill(m->ctx, {batch * c.kv_heads * c.max_ctx, c.head_dim}, kv, 0);
    }
    m->cache_batch = batch;
  }
  if (batch != m->cache_batch) throw burn::Error(MI_E_ARG, "batch differs from the cache's; reset first");
}

}  // namespace

extern "C" {

const char *mi_models_last_error(void) { return g_model_error.c_str(); }

int mi_llama_create(mi_ctx *ctx, const mi_llama_config *cfg, uint64_t seed, float init_std, mi_llama **out) {
  if (!ctx || !cfg || !out) return MI_E_ARG;
  const mi_llama_config &c = *cfg;
  if (c.heads <= 0 || c.kv_heads <= 0 || c.heads % c.kv_heads || c.head_dim % 2 || c.layers < 0 || c.max_ctx <= 0 ||
      c.max_batch <= 0 || (c.numerics != MI_NUMERICS_REFERENCE && c.numerics != MI_NUMERICS_PERFORMANCE)) {
    g_model_error = "invalid llama config";
    return MI_E_ARG;
  }
  mi_llama *m = new mi_llama();
  try {
    m->ctx = ctx;
    m->cfg = c;
    uint64_t base = seed * 1000003ull;
    auto next = [&]() { return base++; };
    const int64_t qd = static_cast<int64_t>(c.heads) * c.head_dim, kvd = static_cast<int64_t>(c.kv_heads) * c.head_dim;
    m->embed = weight(ctx, c.vocab, c.hidden, init_std, next());
    m->final_norm = ones(ctx, c.hidden);
    m->layers.resize(c.layers);
    for (Layer &L : m->layers) {
      L.attn_norm = ones(ctx, c.hidden);
      L.wqkv = weight(ctx, qd + 2 * kvd, c.hidden, init_std, next());
      L.wo = weight(ctx, c.hidden, qd, init_std, next());
      L.mlp_norm = ones(ctx, c.hidden);
      L.wgu = weight(ctx, 2 * static_cast<int64_t>(c.intermediate), c.hidden, init_std, next());
      L.wdown = weight(ctx, c.hidden, c.intermediate, init_std, next());
      if (c.numerics == MI_NUMERICS_PERFORMANCE) {
        // BFP8 (mi_cast_bfp); the BF16 copies become the values it holds.  The
        // decode kernels read BFP8 rows whose width is a multiple of 16; other
        // shapes keep only the BF16 copies of the same values.
        const bool native = c.hidden % 16 == 0 && c.intermediate % 16 == 0 && qd % 16 == 0;
        for (auto wp : {std::make_pair(&L.wqkv, &L.q_wqkv), std::make_pair(&L.wo, &L.q_wo),
                        std::make_pair(&L.wgu, &L.q_wgu), std::make_pair(&L.wdown, &L.q_wdown)}) {
          Tensor held = burn::float_cast(*wp.first, MI_BFP8);
          *wp.first = burn::float_cast(held, MI_BF16);
          if (native) *wp.second = held;
        }
      }
      Tensor pairs;
      if (c.intermediate % 32 == 0 && c.hidden % 32 == 0) {
        const int64_t I = c.intermediate, Hd = c.hidden;
        const int64_t dims[4] = {I / 32, 2, 32, Hd}, st[4] = {32 * Hd, I * Hd, Hd, 1};
        pairs = burn::copy4(L.wgu, dims, 0, st);
        if (I % 128 == 0) L.wgu_pairs = pairs;
      }
      // Tiles: k (hidden, heads x 64, intermediate) a multiple of 16 up to
      // 1536, output widths of 32 (pairs and 64-wide heads of 64).
      if (c.head_dim == 64 && pairs.defined() && qd % 16 == 0 && c.hidden <= 1536 && qd <= 1536 &&
          c.intermediate <= 1536) {
        L.t_wqkv = burn::tile(L.wqkv, MI_TILES_BF16);
        L.t_wo = burn::tile(L.wo, MI_TILES_BF16);
        L.t_wgu_pairs = burn::tile(pairs, MI_TILES_BF16);
        L.t_wdown = burn::tile(L.wdown, MI_TILES_BF16);
      }
    }
    // Rotary tables (rope.rs:14-60): angle = position * theta^(-2i / d), the
    // first half repeated as the second, sin's first half negated.
    const int64_t D = c.head_dim, half = D / 2;
    std::vector<float> cs(static_cast<size_t>(c.max_ctx * D)), sn(cs.size());
    for (int64_t p = 0; p < c.max_ctx; ++p)
      for (int64_t i = 0; i < half; ++i) {
        const float freq = static_cast<float>(std::pow(static_cast<double>(c.rope_theta), -2.0 * i / D));
        const float ang = static_cast<float>(p) * freq;
        const float co = static_cast<float>(std::cos(static_cast<double>(ang)));
        const float si = static_cast<float>(std::sin(static_cast<double>(ang)));
        cs[p * D + i] = co;
        cs[p * D + half + i] = co;
        sn[p * D + i] = -si;
        sn[p * D + half + i] = si;
      }
    m->rope_cos = burn::float_from_data(ctx, cs.data(), {c.max_ctx, D});
    m->rope_sin = burn::float_from_data(ctx, sn.data(), {c.max_ctx, D});
  } catch (const std::exception &e) {
    delete m;
    return fail_model(e);
  }
  *out = m;
  return MI_OK;
}

int mi_llama_destroy(mi_llama *m) {
  if (m) drop_traces(m);
  delete m;
  return MI_OK;
}

int mi_llama_param(mi_llama *m, int layer, int which, mi_id *out) {
  if (!m || !out) return MI_E_ARG;
  const mi_llama_config &c = m->cfg;
  const int64_t qd = static_cast<int64_t>(c.heads) * c.head_dim,
                kvd = static_cast<int64_t>(c.kv_heads) * c.head_dim, I = c.intermediate;
  const Tensor *t = nullptr;
  int64_t row0 = 0, nrows = -1;  // a row block of a fused matrix
  if (which == 0) t = &m->embed;
  else if (which == 1) t = &m->final_norm;
  else if (layer >= 0 && layer < static_cast<int>(m->layers.size())) {
    Layer &L = m->layers[layer];
    switch (which) {
      case 2: t = &L.attn_norm; break;
      case 3: t = &L.wqkv; row0 = 0; nrows = qd; break;
      case 4: t = &L.wqkv; row0 = qd; nrows = kvd; break;
      case 5: t = &L.wqkv; row0 = qd + kvd; nrows = kvd; break;
      case 6: t = &L.wo; break;
      case 7: t = &L.mlp_norm; break;
      case 8: t = &L.wgu; row0 = 0; nrows = I; break;
      case 9: t = &L.wgu; row0 = I; nrows = I; break;
      case 10: t = &L.wdown; break;
      default: break;
    }
  }
  if (!t) {
    g_model_error = "no such parameter";
    return MI_E_ARG;
  }
  try {
    // A copy (of the whole weight or of its row block) the caller frees.
    mi_id id;
    const int64_t cols = t->cols();
    const int64_t n = nrows < 0 ? t->rows() : nrows;
    const int64_t dims[4] = {1, 1, n, cols};
    const int64_t st[4] = {0, 0, cols, 1};
    burn::check(m->ctx, mi_copy_strided4(m->ctx, t->use(), dims, row0 * cols, st, &id), "param");
    *out = id;
  } catch (const std::exception &e) {
    return fail_model(e);
  }
  return MI_OK;
}

int mi_llama_reset(mi_llama *m) {
  if (!m) return MI_E_ARG;
  m->len = 0;
  return MI_OK;
}

int mi_llama_forward(mi_llama *m, const int32_t *ids, int32_t batch, int32_t t, int32_t all_positions,
                     mi_id *logits) {
  if (!m || !ids || !logits || batch <= 0 || t <= 0) return MI_E_ARG;
  try {
    if (batch > m->cfg.max_batch || m->len + t > m->cfg.max_ctx) throw burn::Error(MI_E_ARG, "batch or context too large");
    ensure_cache(m, batch);
    Tensor h = forward_hidden(m, ids, batch, t);
    Tensor out = all_positions ? head_all(m, h) : head_last(m, h, batch, t);
    // Hand the buffer to the caller: it owns (and frees) the id.
    mi_id id;
    burn::check(m->ctx, mi_cast(m->ctx, out.use(), MI_F32, &id), "logits");
    *logits = id;
  } catch (const std::exception &e) {
    return fail_model(e);
  }
  return MI_OK;
}

int mi_llama_generate(mi_llama *m, const int32_t *prompt, int32_t batch, int32_t t_prompt, int32_t n_new,
                      int32_t *out, double *prefill_ms, double *decode_ms) {
  // At least one new token, as the reference's generate_with asserts
  // (crates/tt-models/src/llama.rs:1155): `out` holds batch * n_new tokens.
  if (!m || !prompt || !out || batch <= 0 || t_prompt <= 0 || n_new < 1) return MI_E_ARG;
  using clock = std::chrono::steady_clock;
  try {
    if (batch > m->cfg.max_batch || t_prompt + n_new > m->cfg.max_ctx) throw burn::Error(MI_E_ARG, "batch or context too large");
    m->len = 0;
    ensure_cache(m, batch);
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    auto t0 = clock::now();
    Tensor h = forward_hidden(m, prompt, batch, t_prompt);
    Tensor next = greedy_last(m, h, batch, t_prompt);
    std::vector<int32_t> tok = burn::int_into_data(next);  // waits for the prefill
    auto t1 = clock::now();
    for (int32_t b = 0; b < batch; ++b) out[b * n_new + 0] = tok[b];
    // Each step's tokens stay on the device and feed the next step's
    // embedding gather: no host round trip (and no drained queue) between
    // steps.
    // Each step's tokens go to row s - 1 of one device log, read back with
    // one wait (reading 127 steps' tokens one buffer at a time cost a host
    // round trip each: batch-1 decode 0.564 -> 0.540 ms a step without them,
    // performance contract).
    Tensor log = n_new > 1 ? burn::fill(m->ctx, {n_new - 1, batch}, MI_I32, 0) : Tensor();
    for (int32_t s = 1; s < n_new; ++s) {
      Tensor hs = forward_ids(m, next.reshape({batch}), batch, 1);
      next = greedy_last(m, hs, batch, 1);
      burn::check(m->ctx, mi_assign_block(m->ctx, log.use(), next.reshape({1, batch}).use(), s - 1, 0),
                  "assign_block");
    }
    if (n_new > 1) {
      tok = burn::int_into_data(log);
      for (int32_t s = 1; s < n_new; ++s)
        for (int32_t b = 0; b < batch; ++b) out[b * n_new + s] = tok[static_cast<size_t>(s - 1) * batch + b];
    }
    auto t2 = clock::now();
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  } catch (const std::exception &e) {
    return fail_model(e);
  }
  return MI_OK;
}

}  // extern "C"

namespace {

// The chained decode step's device buffers for `batch` sequences: the input
// token ids, the position of those tokens, the token log.
void step_buffers(mi_llama *m, int64_t batch) {
  mi_ctx *ctx = m->ctx;
  if (!m->step_ids.defined() || m->step_ids.rows() != batch) m->step_ids = burn::fill(ctx, {batch, 1}, MI_I32, 0);
  if (!m->step_pos.defined()) m->step_pos = burn::fill(ctx, {1, 1}, MI_I32, 0);
  if (!m->step_log.defined() || m->step_log.rows() != batch)
    m->step_log = burn::fill(ctx, {batch, m->cfg.max_ctx}, MI_I32, 0);
}

// The decode step of `span`, captured on first use: the token ids and the
// position come from m->step_ids and m->step_pos; the step ends with
// mi_decode_advance, which makes its chosen ids the next step's input, logs
// them at the next position and advances the position -- so replays chain
// on the device, with no host transfer between tokens.  Capture records the
// launches without running them: the caches are not touched.
StepTrace &step_trace(mi_llama *m, int64_t batch, int64_t span) {
  auto it = m->traces.find(span);
  if (it != m->traces.end()) return it->second;
  mi_ctx *ctx = m->ctx;
  step_buffers(m, batch);
  burn::check(ctx, mi_trace_begin(ctx), "trace_begin");
  StepTrace st;
  try {
    Tensor x = burn::select_rows_as(m->embed, m->step_ids.reshape({batch}), MI_F32);
    x = decode_layers(m, x.reshape({batch, m->cfg.hidden}), batch, &m->step_pos, 0, span);
    st.next = greedy_last(m, x, batch, 1);
    burn::check(ctx, mi_decode_advance(ctx, st.next.use(), m->step_ids.use(), m->step_pos.use(), m->step_log.use()),
                "decode_advance");
  } catch (...) {
    uint64_t dead = 0;
    if (mi_trace_end(ctx, &dead) == MI_OK) (void)mi_trace_release(ctx, dead);
    throw;
  }
  burn::check(ctx, mi_trace_end(ctx, &st.id), "trace_end");
  return m->traces[span] = std::move(st);
}

// The prefill of `t` tokens per sequence into the empty caches, captured on
// first use (the reference's traced prompt chunk): embedding gather, the
// layers, the head on each sequence's last position and the argmax.  A path
// that cannot be captured leaves a record with id 0.
PromptTrace &prompt_trace(mi_llama *m, int64_t batch, int64_t t) {
  const auto key = std::make_pair(batch, t);
  auto it = m->prompt_traces.find(key);
  if (it != m->prompt_traces.end()) return it->second;
  mi_ctx *ctx = m->ctx;
  PromptTrace pt;
  pt.ids = burn::fill(ctx, {batch * t}, MI_I32, 0);
  burn::check(ctx, mi_trace_begin(ctx), "trace_begin");
  try {
    m->len = 0;
    Tensor h = forward_ids(m, pt.ids, batch, t);
    pt.next = greedy_last(m, h, batch, t);
    m->len = 0;  // the capture ran nothing
  } catch (const burn::Error &e) {
    m->len = 0;
    uint64_t dead = 0;
    if (mi_trace_end(ctx, &dead) == MI_OK) (void)mi_trace_release(ctx, dead);
    if (e.status != MI_E_UNSUPPORTED) throw;
    PromptTrace eager;
    return m->prompt_traces[key] = std::move(eager);
  } catch (...) {
    m->len = 0;
    uint64_t dead = 0;
    if (mi_trace_end(ctx, &dead) == MI_OK) (void)mi_trace_release(ctx, dead);
    throw;
  }
  burn::check(ctx, mi_trace_end(ctx, &pt.id), "trace_end");
  return m->prompt_traces[key] = std::move(pt);
}

}  // namespace

extern "C" int mi_llama_generate_traced(mi_llama *m, const int32_t *prompt, int32_t batch, int32_t t_prompt,
                                        int32_t n_new, int32_t *out, double *prefill_ms, double *decode_ms) {
  if (!m || !prompt || !out || batch <= 0 || t_prompt <= 0 || n_new < 1) return MI_E_ARG;
  if (!decode_fused(m, batch))  // no fused decode step to capture: the eager loop
    return mi_llama_generate(m, prompt, batch, t_prompt, n_new, out, prefill_ms, decode_ms);
  using clock = std::chrono::steady_clock;
  try {
    if (batch > m->cfg.max_batch || t_prompt + n_new > m->cfg.max_ctx) throw burn::Error(MI_E_ARG, "batch or context too large");
    m->len = 0;
    ensure_cache(m, batch);
    burn::check(m->ctx, mi_sync(m->ctx), "sync");
    // The prompt: a replay of its captured prefill (ids in), or eagerly where
    // the prefill cannot be captured; its first new ids start the chain.
    PromptTrace &pt = prompt_trace(m, batch, t_prompt);
    step_buffers(m, batch);
    mi_ctx *ctx = m->ctx;
    const Tensor start = burn::fill(ctx, {1, 1}, MI_I32, static_cast<uint32_t>(t_prompt - 1));
    auto t0 = clock::now();
    Tensor first;
    if (pt.id) {
      const mi_id in_ids[1] = {pt.ids.id()};
      const void *in_vals[1] = {prompt};
      const int64_t in_len[1] = {static_cast<int64_t>(batch) * t_prompt * 4};
      burn::check(ctx, mi_trace_run(ctx, pt.id, 1, in_ids, in_vals, in_len, 0, nullptr, nullptr, nullptr),
                  "trace_run");
      first = pt.next;
    } else {
      Tensor h = forward_hidden(m, prompt, batch, t_prompt);
      first = greedy_last(m, h, batch, t_prompt);
    }
    m->len = t_prompt;
    // The first ids are the input at position t_prompt: the chain starts one
    // before it, and mi_decode_advance logs them there and moves on.
    burn::check(ctx, mi_copy_into(ctx, start.use(), m->step_pos.use()), "copy_into");
    burn::check(ctx, mi_decode_advance(ctx, first.use(), m->step_ids.use(), m->step_pos.use(), m->step_log.use()),
                "decode_advance");
    burn::check(ctx, mi_sync(ctx), "sync");
    auto t1 = clock::now();
    // Each later token: one replay of the step for its span, queued behind
    // the last with no transfer; the tokens come back once, at the end.
    for (int32_t s = 1; s < n_new; ++s) {
      StepTrace &st = step_trace(m, batch, decode_span(m, m->len + 1));
      burn::check(ctx, mi_trace_run(ctx, st.id, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr),
                  "trace_run");
      m->len += 1;
    }
    const std::vector<int32_t> log = burn::int_into_data(m->step_log);  // waits for the last step
    const int64_t cols = m->cfg.max_ctx;
    for (int32_t b = 0; b < batch; ++b)
      for (int32_t s = 0; s < n_new; ++s) out[b * n_new + s] = log[static_cast<size_t>(b * cols + t_prompt + s)];
    auto t2 = clock::now();
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  } catch (const std::exception &e) {
    return fail_model(e);
  }
  return MI_OK;
}
