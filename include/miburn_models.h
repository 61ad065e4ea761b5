/*
 * miburn_models.h -- the model harnesses that drive the engine: the callers
 * on either side of the hot path (the reference's crates/tt-mnist and
 * crates/tt-models), written once over the engine's C ABI (miburn.h).
 * They are not part of the engine boundary; tests and bench.py reach them
 * through these entry points.
 */
#ifndef MIBURN_MODELS_H
#define MIBURN_MODELS_H

#include <stdint.h>

#include "miburn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Llama / SmolLM2 decoder (crates/tt-models/src/llama.rs:40-71,
 * 140-520, 1030-1178): pre-norm GQA attention with RoPE, SwiGLU MLP, RMSNorm,
 * tied embedding head, BF16 weights and F32 activations. ---- */

/* The two numeric contracts inference runs under (llama.rs:1252-1282, the
 * reference's `Numerics`): REFERENCE keeps the KV cache and every
 * activation F32; PERFORMANCE stores the KV cache BF16 (half its bytes) and
 * rounds each activation a prefill's product reads to BF16 once, where it is
 * made (the attention and MLP norms, the attention output, the SiLU-mul, the
 * final norm).  A decode step's fused projections read F32 activations under
 * both: their traffic is the weights'.  The reference's BFP8 weights are a
 * Tensix block format with no counterpart here; weights are BF16 under both. */
#define MI_NUMERICS_REFERENCE 0
#define MI_NUMERICS_PERFORMANCE 1

typedef struct mi_llama_config {
  int32_t vocab, hidden, layers, heads, kv_heads, head_dim, intermediate;
  float rope_theta, eps;
  int32_t max_ctx, max_batch;
  int32_t numerics; /* MI_NUMERICS_* */
} mi_llama_config;

typedef struct mi_llama mi_llama;

/* Random init: every weight N(0, init_std^2) drawn on the device from `seed`
 * and stored BF16; RMSNorm gains 1. */
int mi_llama_create(mi_ctx *ctx, const mi_llama_config *cfg, uint64_t seed,
                    float init_std, mi_llama **out);
int mi_llama_destroy(mi_llama *m);
/* A copy of a weight (for checks), a new id the caller frees: which = 0
 * embedding table [vocab, hidden] (layer ignored), 1 final norm; per layer
 * 2 attention norm, 3 q [q_dim, hidden], 4 k [kv_dim, hidden], 5 v, 6 o
 * [hidden, q_dim], 7 mlp norm, 8 gate [inter, hidden], 9 up, 10 down
 * [hidden, inter].  Projection weights are stored [out, in] (the product
 * reads them transposed); q|k|v and gate|up are row blocks of one fused
 * matrix each. */
int mi_llama_param(mi_llama *m, int layer, int which, mi_id *out);
/* Empty the KV cache. */
int mi_llama_reset(mi_llama *m);
/* Feed `t` tokens per sequence (ids [batch, t], row-major) at the cache's
 * current length; return the logits of every position ([batch * t, vocab],
 * all_positions != 0) or of each sequence's last ([batch, vocab]). */
int mi_llama_forward(mi_llama *m, const int32_t *ids, int32_t batch,
                     int32_t t, int32_t all_positions, mi_id *logits);
/* Greedy generation (llama.rs:1136-1178): prefill the prompts, then decode
 * n_new tokens per sequence, each the argmax of the last logits.  `out`
 * receives [batch, n_new] ids; the times (ms, device-synchronised) of the
 * prefill and of all decode steps are returned if the pointers are set. */
int mi_llama_generate(mi_llama *m, const int32_t *prompt, int32_t batch,
                      int32_t t_prompt, int32_t n_new, int32_t *out,
                      double *prefill_ms, double *decode_ms);
/* mi_llama_generate with the prompt and each decode step trace replays
 * (the reference's TracedGenerator, crates/tt-models/src/generate.rs:1-22,
 * 770-790): the prefill is captured once per (batch, prompt length), token
 * ids in and the first new ids out (eager where its path cannot be captured:
 * the composition's causal mask is an upload); the decode step is captured
 * once per span of 64 attended positions over the model's caches and
 * replayed per token, the token ids and the position written into the
 * trace's inputs and the next ids read back.  The tokens equal
 * mi_llama_generate's bit for bit (the eager steps run the same launches).
 * Traces live until the caches are reallocated (a new batch size) or the
 * model is destroyed.  A batch the fused decode step does not take runs
 * mi_llama_generate. */
int mi_llama_generate_traced(mi_llama *m, const int32_t *prompt, int32_t batch,
                             int32_t t_prompt, int32_t n_new, int32_t *out,
                             double *prefill_ms, double *decode_ms);

/* Last error message of the model layer. */
const char *mi_models_last_error(void);

/* ---- MLP d_in -> hidden -> d_out, ReLU, softmax cross-entropy, SGD (the
 * reference's MNIST gate, crates/tt-tests/tests/step12_mnist.rs:57-114):
 * Burn `Linear` layers, weight [d_in, d_out], initialised U(-k, k),
 * k = 1/sqrt(d_in), from the gate's 64-bit LCG seeded `lcg_seed`. ---- */
typedef struct mi_mlp mi_mlp;
int mi_mlp_create(mi_ctx *ctx, int32_t d_in, int32_t hidden, int32_t d_out,
                  uint64_t lcg_seed, mi_mlp **out);
int mi_mlp_destroy(mi_mlp *m);
/* which: 0 w1 [d_in, hidden], 1 b1 [1, hidden], 2 w2 [hidden, d_out], 3 b2. */
int mi_mlp_param(mi_mlp *m, int which, mi_id *out);
/* One step on resident x [B, d_in] F32 and labels (B I32): forward, loss,
 * backward, SGD update; the loss [1, 1] is a new id the caller frees. */
int mi_mlp_train_step(mi_mlp *m, mi_id x, mi_id labels, float lr, mi_id *loss);
/* `steps` steps on device-drawn data (x ~ U[0, 1), labels uniform in
 * [0, d_out)); per-step losses and the wall time of all steps (ms, synced). */
int mi_mlp_train_synthetic(mi_mlp *m, int32_t batch, int32_t steps, float lr,
                           uint64_t data_seed, float *losses, double *ms);
const char *mi_mlp_last_error(void);

/* ---- Transformer training (the reference's TinyTransformer,
 * crates/tt-mnist/src/transformer.rs:36-166, trained by
 * crates/tt-tests/tests/step59_burn_transformer.rs): Embedding, pre-norm
 * encoder layers (LayerNorm, multi-head self-attention without a mask,
 * LayerNorm, Linear-GELU-Linear), Linear head, cross-entropy, SGD; F32.
 * Burn's default init drawn on the device from `seed`: embedding N(0, 1),
 * Linear weight [d_in, d_out] and bias U(-1/sqrt(d_in), 1/sqrt(d_in)),
 * LayerNorm gamma 1, beta 0. ---- */
typedef struct mi_transformer_config {
  int32_t vocab, d_model, heads, d_ff, layers;
  float eps;
} mi_transformer_config;

typedef struct mi_transformer mi_transformer;
int mi_transformer_create(mi_ctx *ctx, const mi_transformer_config *cfg,
                          uint64_t seed, mi_transformer **out);
int mi_transformer_destroy(mi_transformer *m);
/* layer < 0: which 0 embedding [vocab, d], 1 head weight [d, vocab], 2 head
 * bias [1, vocab].  layer >= 0: which 0 ln1 gamma, 1 ln1 beta, 2 wq, 3 bq,
 * 4 wk, 5 bk, 6 wv, 7 bv, 8 wo, 9 bo (weights [d, d], biases [1, d]),
 * 10 ln2 gamma, 11 ln2 beta, 12 w1 [d, d_ff], 13 b1, 14 w2 [d_ff, d], 15 b2.
 * The result is a copy, a new id the caller frees (q, k and v are column
 * blocks of one fused weight inside the model). */
int mi_transformer_param(mi_transformer *m, int layer, int which, mi_id *out);
/* One step on resident tokens and targets (batch * seq I32 each, row-major
 * [batch, seq]): forward, mean cross-entropy over all positions, backward,
 * SGD with rate lr.  The loss [1, 1] is a new id the caller frees. */
int mi_transformer_train_step(mi_transformer *m, mi_id tokens, mi_id targets,
                              int32_t batch, int32_t seq, float lr,
                              mi_id *loss);
/* `steps` steps on device-drawn tokens and targets, each uniform in
 * [0, vocab); per-step losses and the wall time of all steps (ms, synced). */
int mi_transformer_train_synthetic(mi_transformer *m, int32_t batch,
                                   int32_t seq, int32_t steps, float lr,
                                   uint64_t data_seed, float *losses,
                                   double *ms);
const char *mi_transformer_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* MIBURN_MODELS_H */
