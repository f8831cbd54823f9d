/*
 * TEST INFRASTRUCTURE ONLY — not part of the product.
 *
 * CPU restatement of the reference Mesh GPT forward pass and its `generate`
 * loop, in plain C with f64 arithmetic.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load this library, and only as the
 * checker or the timed CPU baseline; the product library never links it.
 *
 * The reference is pure Rust (/root/reference/src/gpt/); no Rust toolchain
 * exists in this image, so nothing of it can be built (oracle/_ref stays empty).
 * Each function below names the reference lines it restates.  How each one is
 * pinned (reference KATs, published whole-model numbers, closed forms,
 * independent numpy restatements) is recorded in tests/test_oracle.py.
 * og_sample with temperature > 0 has no reference vector; it is pinned by
 * closed forms, an exact rescaling symmetry and its realised distribution.
 */
#ifndef MESHGPT_ORACLE_H
#define MESHGPT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GptConfig (reference src/gpt/config.rs:21-56) with its operator switches
 * (config.rs:33-35) and EmbeddingGeometry (geometry.rs:49-81); codes as in the
 * checkpoint (checkpoint.rs:146-168). */
typedef struct {
    uint32_t vocab_size;
    uint32_t context;
    uint32_t width;
    uint32_t heads;
    uint32_t layers;
    uint32_t attention_mesh_depth;
    uint32_t ffn_mesh_depth;
    uint32_t embedding;    /* 0 = mesh (default), 1 = table (config.rs:58-67) */
    uint32_t connectivity; /* 0 = neighbor (default), 1 = butterfly (config.rs:96-106) */
    uint32_t rope, qk_norm, xsa; /* 1 = on (default) */
    uint32_t form;          /* 0 parity (default) .. 9 sphere, geometry.rs:37-41 */
    uint32_t order;         /* 0 token (default), 1 residue, 2 discrete-log */
    uint32_t frequency;     /* default 1 */
    uint32_t harmonics;     /* default 1 */
    float overlap;
    uint32_t normalization; /* 0 none (default), 1 unit, 2 rms */
    uint32_t frozen;
    uint32_t preserve_features;
    uint32_t modulus;
    uint64_t seed;
} og_config;

/* ---- SplitMix64 (reference src/mesh.rs:256-288) ---- */
uint64_t og_rng_next(uint64_t *state);
float og_rng_unit(uint64_t *state);
uint64_t og_rng_index(uint64_t *state, uint64_t bound);

/* ---- configuration, layout, initialisation (config.rs:117-122,144-172,358-459) ---- */
/* Returns 0 when valid, else writes the reference's message into err (may be NULL). */
int og_validate(const og_config *c, int allow_long_context, char *err, size_t err_len);
size_t og_parameter_count(const og_config *c);
size_t og_embedding_parameter_count(const og_config *c);
/* offset of each parameter group: [0] embedding, then per block q,k,v,proj,ffn */
void og_group_offsets(const og_config *c, size_t *offsets /* 1+5L */);
uint32_t og_stride(const og_config *c, uint32_t layer);
void og_initialize(const og_config *c, uint64_t seed, float *out);
void og_initialize_normal(const og_config *c, uint64_t seed, float sigma, float *out);
/* fixed token codes, V x W (config.rs:552-591, geometry.rs:186-325) */
void og_token_codes(const og_config *c, float *out);
/* grokking.rs:260-271 (modulus entries) and geometry.rs:166-184 */
void og_residue_permutation(uint32_t modulus, uint64_t seed, uint32_t *out);
uint32_t og_primitive_root(uint32_t prime);

/* ---- per-op references used by the reference's own KATs (reference.rs:392-603) ---- */
void og_rmsnorm(const double *in, size_t width, size_t heads, double *out);
void og_rotary(const double *in, size_t width, size_t heads, size_t position, double *out);
void og_exclusive(const double *y, const double *v, size_t width, size_t heads, double *out);
/* rows x width q,k,v; causal attention inside consecutive sequences of `sequence` rows */
void og_attention(const double *q, const double *k, const double *v, size_t rows, size_t width,
                  size_t heads, size_t sequence, double *out);
/* a mesh stack over rows x width; params points at the group's first weight */
void og_mesh(const double *in, size_t rows, size_t width, const float *params, size_t depth,
             uint32_t connectivity, double *out);

/* ---- whole model (reference.rs:49-59,90-102,104-228) ---- */
/* effective token vectors, V x W */
int og_token_embeddings(const og_config *c, const float *params, double *out);
/* logits for every row, n x V (f64, before the f32 cast of reference.rs:54) */
int og_logits(const og_config *c, const float *params, const uint32_t *tokens, size_t n,
              size_t sequence, double *out);
/* residual stream before the final RMSNorm, n x W */
int og_hidden_states(const og_config *c, const float *params, const uint32_t *tokens, size_t n,
                     size_t sequence, double *out);
/* next-token cross-entropy, mean over rows whose target != UINT32_MAX, computed on the
 * f32-cast logits like the reference's loss kernel (gpu.rs:949-994,2296-2313) */
int og_cross_entropy(const og_config *c, const float *params, const uint32_t *inputs,
                     const uint32_t *targets, size_t n, size_t sequence, double *loss);

/* ---- training (meshgpt_oracle_grad.c) ---- */
/* the gradient mask's range of group `group` (config.rs:461-474), as offsets in the group */
void og_constrained_range(const og_config *c, size_t group, size_t *begin, size_t *end);
/* reference.rs:61-89: mean next-token cross-entropy over rows whose target != UINT32_MAX and
 * its gradient (og_parameter_count entries, masked as config.rs:490-500), by reverse
 * accumulation over the reference's scalar tape.  0 on success; -1 invalid inputs, -3 a
 * target outside the vocabulary, -4 no supervised target, -5 non-finite, -6 out of memory. */
int og_loss_and_gradient(const og_config *c, const float *params, const uint32_t *inputs,
                         const uint32_t *targets, size_t n, size_t sequence, double *loss, double *gradient);
/* one f32 AdamW update (gpu.rs:1366-1391) of `count` parameters with moments m, v and the
 * step's bias corrections 1 - beta^t */
void og_adam(float *value, float *m, float *v, const float *gradient, size_t count, float learning_rate,
             float weight_decay, float beta1, float beta2, float epsilon, float correction1, float correction2);

/* ---- generate (reference src/gpt/gpu.rs:2006-2053) ----
 * prompt of P tokens; writes P+count tokens into out.  Every step recomputes the
 * window of at most `context` tokens, exactly as the reference does. */
int og_generate(const og_config *c, const float *params, const uint32_t *prompt, size_t P,
                size_t count, float temperature, uint64_t seed, uint32_t *out);
/* the f32 sampler of gpu.rs:2028-2049 on one row of f32 logits; returns the token and
 * advances *rng only when temperature > 0 */
uint32_t og_sample(const float *logits, size_t vocab, float temperature, uint64_t *rng);

/* ---- KV-cached incremental decode (same math, used as the CPU baseline) ----
 * Valid while P+count <= context; returns -1 otherwise. */
int og_generate_cached(const og_config *c, const float *params, const uint32_t *prompt, size_t P,
                       size_t count, float temperature, uint64_t seed, uint32_t *out,
                       float *last_logits /* V, may be NULL */);

/* ---- datasets used by the published-number pins ---- */
/* TextDataset::batch (src/gpt/text.rs:63-108) over an already tokenised corpus */
int og_text_batch(const uint32_t *tokens, size_t len, int validation, size_t sequence,
                  size_t batch, uint64_t seed, uint32_t *inputs, uint32_t *targets);
/* EquationDataset (src/gpt/grokking.rs:116-186,228-271): writes the residue permutation
 * (p entries) and both splits as (a,b,answer) triples; returns the training count. */
int og_equations(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed,
                 uint32_t *residue_tokens, uint32_t *train /* 3*n */, uint32_t *valid /* 3*n */,
                 size_t *n_train, size_t *n_valid);
/* row_metrics of src/bin/mesh-gpt/grokking.rs:544-557 on one f32 row */
double og_row_metrics(const float *row, size_t vocab, size_t target, size_t *prediction);

/* ---- CPU baseline (bench.py's cpu_baseline leg; cpu_f32_decode.c) ----
 * KV-cached f32 decode on `threads` OpenMP threads, one sequence a thread:
 * prompts B x P, then `steps` decode steps (the forward of the last token and
 * the draw of the next, seed + b per sequence, og_sample's arithmetic);
 * out: B x (P + steps + 1) tokens; decode_seconds: wall time of the steps.
 * Returns nonzero for shapes it does not take (geometric forms, embedding
 * normalisation, protected coordinates, P + steps beyond the context). */
int cb_generate_f32(const og_config *c, const float *params, const uint32_t *prompts, size_t B, size_t P,
                    size_t steps, float temperature, uint64_t seed, int threads, uint32_t *out,
                    double *decode_seconds);

#ifdef __cplusplus
}
#endif

#endif
