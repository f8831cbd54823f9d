/*
 * meshgpt.h — C ABI of the MI355X Mesh GPT generate path (libmeshgpt.so).
 *
 * This is the seam that replaces the reference's cuda-oxide launcher and the
 * Rust `SpecializedMeshGpt` inference API (src/gpt/gpu.rs:21-1392 kernels and
 * launcher, 1693-2092 public API).  Plain C types only: an opaque model handle,
 * caller-owned host buffers, an int status and a thread-local message that
 * carries the reference's error text.  Every call returns after its work is
 * complete on the device; calls on one handle must not overlap (the caller
 * serialises them, as the reference's &self / &mut self borrows do);
 * distinct handles are independent.  All host pointers are borrowed for the
 * duration of the call only.
 */
#ifndef MESHGPT_H
#define MESHGPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The message of the last failure on the calling thread is
 * returned by mg_last_error(). */
enum {
    MG_OK = 0,
    MG_INVALID_ARGUMENT = 1, /* the reference's Err(...) on validation */
    MG_OUT_OF_MEMORY = 2,
    MG_DEVICE_ERROR = 3,
    MG_NONFINITE = 4, /* "... must contain only finite values" (src/mesh.rs:239-246) */
    MG_IO = 5,        /* checkpoint files */
    MG_UNSUPPORTED = 6 /* MSHGPT09 geometry/operator ablations */
};

/* GptConfig (src/gpt/config.rs:21-56) in checkpoint field order
 * (src/gpt/checkpoint.rs:51-78,129-168).  mg_config_default() gives the
 * reference's defaults: default geometry and RoPE, QK-Norm and XSA on, as in
 * every MSHGPT07/08 checkpoint; MSHGPT09 checkpoints change the rest. */
typedef struct {
    uint32_t vocab_size;
    uint32_t context;
    uint32_t width;
    uint32_t heads;
    uint32_t layers;
    uint32_t attention_mesh_depth;
    uint32_t ffn_mesh_depth;
    uint32_t embedding;    /* 0 mesh, 1 table (config.rs:58-67) */
    uint32_t connectivity; /* 0 neighbor, 1 butterfly (config.rs:96-106) */
    uint32_t long_context; /* extension: 1 accepts context up to 65536 (reference cap 4096,
                              config.rs:148); such configs cannot be checkpointed */
    /* Operator switches (config.rs:33-35): 1 on, 0 off. */
    uint32_t rope;
    uint32_t qk_norm;
    uint32_t xsa;
    /* EmbeddingGeometry (geometry.rs:49-81) with its checkpoint codes: form 0 parity,
     * 1 circle, 2 fourier, 3 orthogonal, 4 simplex, 5 equiangular, 6 antipodal,
     * 7 hypercube, 8 signed-permutations, 9 sphere; order 0 token, 1 residue,
     * 2 discrete-log; normalization 0 none, 1 unit, 2 rms. */
    uint32_t form;
    uint32_t order;
    uint32_t frequency;
    uint32_t harmonics;
    float overlap;
    uint32_t normalization;
    uint32_t frozen;
    uint32_t preserve_features;
    uint32_t modulus;
    uint64_t seed;
} mg_config;

typedef struct mg_model mg_model;

/* Message of the last failed call on this thread ("" if none). */
const char *mg_last_error(void);

/* GptConfig::default() (config.rs:38-55). */
void mg_config_default(mg_config *out);
/* GptConfig::validate (config.rs:144-172). */
int mg_config_validate(const mg_config *config);
/* GptConfig::parameter_count (config.rs:174-176). */
int mg_parameter_count(const mg_config *config, size_t *out);
/* GptConfig::initial_parameters (config.rs:187-190); out holds parameter_count floats. */
int mg_initial_parameters(const mg_config *config, uint64_t seed, float *out, size_t n);
/* No counterpart in config.rs: the N(0, sigma^2) weights of BASELINE.json's
 * synthetic workloads (sigma 0.5 there).  Parameter i, in the flat order of
 * mg_initial_parameters, is sigma times one draw of the reference's Box-Muller
 * normal (src/simple/numerical.rs:163-167) from Random::new(seed) (two unit()
 * draws per parameter); the protected rows of a geometry with
 * preserve_features stay zero.  out holds parameter_count floats. */
int mg_normal_parameters(const mg_config *config, uint64_t seed, float sigma, float *out, size_t n);
/* GptConfig::fixed_token_codes (config.rs:205-208); out is vocab_size x width. */
int mg_token_codes(const mg_config *config, float *out, size_t n);

/* SpecializedMeshGpt::new (gpu.rs:1718-1771): seeded weights on `device`, decode
 * state for max_batch sequences (grown on demand). */
int mg_model_create(int device, const mg_config *config, uint64_t seed, size_t max_batch, mg_model **out);
void mg_model_destroy(mg_model *model);
/* SpecializedMeshGpt::config (gpu.rs:1773-1775). */
int mg_model_config(const mg_model *model, mg_config *out);
/* SpecializedMeshGpt::parameters (gpu.rs:1846-1853). */
int mg_parameters(mg_model *model, float *out, size_t n);
/* SpecializedMeshGpt::set_parameters (gpu.rs:1856-1872). */
int mg_set_parameters(mg_model *model, const float *values, size_t n);
/* SpecializedMeshGpt::logits / cached_logits (gpu.rs:1875-1901): n tokens in
 * sequences of `sequence`; out is n x vocab_size, or (n/sequence) x vocab_size of
 * each sequence's last row when last_only != 0. */
int mg_logits(mg_model *model, const uint32_t *tokens, size_t n, size_t sequence, int last_only,
              float *out, size_t out_len);
/* AdamWOptions (config.rs:258-276); mg_adamw_default fills the reference's
 * defaults (learning rate 0.003, weight decay 0.01, betas 0.9 and 0.999,
 * epsilon 1e-8). */
typedef struct {
    float learning_rate;
    float weight_decay;
    float beta1;
    float beta2;
    float epsilon;
} mg_adamw;
void mg_adamw_default(mg_adamw *out);
/* Target id of a row without supervision (IGNORE_TARGET, src/gpt/mod.rs:26). */
#define MG_IGNORE_TARGET 0xFFFFFFFFu
/* SpecializedMeshGpt::cross_entropy (gpu.rs:1915-1929): the mean next-token
 * cross-entropy over rows whose target is not MG_IGNORE_TARGET; n inputs and
 * n targets in sequences of `sequence`. */
int mg_cross_entropy(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                     double *loss);
/* SpecializedMeshGpt::loss_and_gradient (gpu.rs:1931-1946): the loss and the
 * gradient of every parameter (n_gradient = the parameter count), masked as
 * config.rs:490-500.  The reference returns the f32 gradient widened to f64;
 * this returns the f32 values. */
int mg_loss_and_gradient(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n,
                         size_t sequence, double *loss, float *gradient, size_t n_gradient);
/* SpecializedMeshGpt::train_batch_with_optimizer (gpu.rs:1950-2003): the loss
 * before one AdamW update; the moments and step count persist across calls
 * until mg_set_parameters resets them. */
int mg_train_batch(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                   const mg_adamw *options, double *loss);
/* EquationDataset::new (grokking.rs:128-186): the split sizes of the seeded
 * table of `operation` (ModularOperation order: 0 add, 1 multiply, 2 subtract,
 * 3 divide, 4 mixed, 5 square-sum, 6 quadratic, 7 quadratic-linear, 8
 * cubic-product, 9 cubic-mixed) modulo the prime `modulus`. */
int mg_equation_split(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed, size_t *n_train,
                      size_t *n_valid);
/* EquationDataset::batch (grokking.rs:225-258): 4 * n inputs (a, op, b, '=')
 * and targets (MG_IGNORE_TARGET but the answer) for the split's equations. */
int mg_equation_batch(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed, int validation,
                      const size_t *indices, size_t n, uint32_t *inputs, uint32_t *targets);
/* TextDataset::new + batch (src/gpt/text.rs:63-108): the corpus `tokens` split
 * 90/10 (checked against `config`'s vocabulary and context), then `batch`
 * windows of `sequence` tokens from the training (validation = 0) or
 * validation split at starts drawn from `seed`; targets are the inputs shifted
 * by one.  inputs and targets hold batch * sequence tokens each. */
int mg_text_batch(const uint32_t *tokens, size_t n_tokens, const mg_config *config, int validation,
                  size_t sequence, size_t batch, uint64_t seed, uint32_t *inputs, uint32_t *targets);
/* SpecializedMeshGpt::token_embeddings (gpu.rs:2056-2068): vocab_size x width. */
int mg_token_embeddings(mg_model *model, float *out, size_t n);
/* SpecializedMeshGpt::hidden_states (gpu.rs:2070-2092): n x width. */
int mg_hidden_states(mg_model *model, const uint32_t *tokens, size_t n, size_t sequence, float *out,
                     size_t out_len);

/* SpecializedMeshGpt::generate (gpu.rs:2006-2053) on token ids, batched:
 * prompts is batch x prompt_len, out is batch x (prompt_len + count).  Row b
 * samples with Random::new(seed + b); row 0 is exactly the reference's call. */
int mg_generate(mg_model *model, const uint32_t *prompts, size_t batch, size_t prompt_len, size_t count,
                float temperature, uint64_t seed, uint32_t *out);
/* The same on text: the tokenizer is given as its characters (Unicode scalar
 * values, CharacterTokenizer, src/gpt/text.rs:7-56); prompt is UTF-8.  Writes the
 * UTF-8 result (prompt + generated, no terminator) and its byte length. */
int mg_generate_text(mg_model *model, const uint32_t *characters, size_t vocab, const char *prompt,
                     size_t count, float temperature, uint64_t seed, char *out, size_t capacity,
                     size_t *written);

/* Step-wise decode for benchmarks (no reference counterpart: the reference
 * recomputes the window per token).  mg_prefill runs the prompts and samples
 * the first token; mg_decode runs `steps` more on-device decode steps. */
int mg_prefill(mg_model *model, const uint32_t *prompts, size_t batch, size_t prompt_len, float temperature,
               uint64_t seed, size_t reserve);
int mg_decode(mg_model *model, size_t steps);
/* As mg_decode, without graph replay, timing each decode-attention launch with
 * HIP events on the model's stream: ms has steps x layers entries. */
int mg_decode_profiled(mg_model *model, size_t steps, float *ms, size_t n);
/* As mg_decode, in one persistent launch that records its timeline (no
 * reference counterpart: a profiling aid).  stamps receives blocks x steps x
 * (layers + 1) x 2 wall-clock values at 100 MHz: for each block (3*batch mesh
 * teams, then batch*heads attention blocks), step and phase, when the phase's
 * inputs were ready and when its outputs were published.  Fails with
 * MG_UNSUPPORTED when the persistent kernel cannot run this model and batch. */
int mg_decode_traced(mg_model *model, size_t steps, uint64_t *stamps, size_t n);
/* Restores the decode state that the last mg_prefill left: every sequence's
 * length and sampler state (no reference counterpart: it lets a benchmark
 * repeat the same decode steps from resident inputs).  The cache rows of the
 * prompts stay valid; rows of later positions are rewritten by the next
 * decode.  Two small device copies on the model's stream; nothing is
 * allocated. */
int mg_decode_rewind(mg_model *model);
/* Device time in milliseconds of the kernels of the last mg_logits,
 * mg_hidden_states or mg_prefill call on this model, or of the last
 * persistent decode launch (mg_decode, mg_generate) (HIP events on the
 * model's stream around its kernels; host copies excluded).  No reference
 * counterpart: it lets a benchmark time a prefill without the PCIe copies and
 * a decode launch without the host's synchronisation. */
int mg_last_call_ms(mg_model *model, float *ms);
/* Current tokens per sequence (prompt + generated). */
int mg_sequence_length(const mg_model *model, size_t *out);
int mg_read_tokens(mg_model *model, uint32_t *out, size_t batch, size_t length);
/* Logits of the last sampled step, batch x vocab_size. */
int mg_last_logits(mg_model *model, float *out, size_t n);
/* The hipStream_t every call of this model runs on. */
void *mg_model_stream(mg_model *model);

/* The sampler of mg_generate (gpu.rs:2028-2049) on `device`, for `rows` rows
 * of `vocab` f32 logits: the first maximal logit when temperature == 0, else
 * one Random::unit() draw from rng_states[r] per row (states advanced in place)
 * and the reference's sequential f32 CDF scan.  Returns MG_NONFINITE (tokens
 * still written) when a row holds a non-finite logit.  No separate reference
 * call: it exposes generate's sampling step to tests. */
int mg_sample_logits(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                     uint64_t *rng_states, uint32_t *tokens);

/* No counterpart in the reference: an entry point for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops).  It is
 * mg_sample_logits on buffers already on `device`: logits (rows x vocab f32),
 * rng_states (rows, advanced in place when temperature > 0) and tokens (rows,
 * written) are device pointers the caller owns, and *nonfinite (a device int)
 * receives 1 when a row holds a non-finite logit, else 0.  The work is
 * enqueued on `stream` (a hipStream_t; NULL is the default stream) and the
 * call returns without waiting.  It allocates nothing: its only scratch is one
 * counter per row in a fixed array of MG_NOALLOC_MAX_ROWS ints on each GPU,
 * held until the process ends, which every call clears before use.  More rows
 * are rejected with MG_INVALID_ARGUMENT.  Calls that overlap on one GPU share
 * that array and race: order them (one stream, or events).  The first call on
 * a device looks up the array's device address (hipGetSymbolAddress); make it
 * before capturing a stream.  The calling thread's current device is the same
 * on return as on entry. */
#define MG_NOALLOC_MAX_ROWS 65536
int mg_sample_logits_noalloc(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                             uint64_t *rng_states, uint32_t *tokens, int *nonfinite, void *stream);

/* out[i] = the f32 exp the sampler of mg_generate uses (the reference's
 * f32::exp, i.e. the C library's expf), evaluated on `device`.  No separate
 * reference call: it lets tests compare the device exp with the host's. */
int mg_expf(int device, const float *x, size_t n, float *out);

/* A plain device-to-device copy of `bytes` (a float4 grid-stride kernel named
 * calibration_copy) run `iters` times on `device`; writes the mean bandwidth
 * counting read plus write bytes.  No reference counterpart: it calibrates the
 * HBM byte counters and gives the measured copy roofline of the box. */
int mg_copy_bandwidth(int device, size_t bytes, int iters, double *gbps);

/* CharacterTokenizer (src/gpt/text.rs:7-56).  A tokenizer is passed as its
 * characters (Unicode scalar values, token id = index).
 * mg_tokenizer_from_text (text.rs:13-15): the sorted unique characters of the
 * UTF-8 text; *n receives their count, and characters may be NULL to query it.
 * mg_tokenizer_encode (text.rs:30-43): UTF-8 text -> token ids, *n = count.
 * mg_tokenizer_decode (text.rs:45-55): token ids -> UTF-8 (no terminator),
 * *written = bytes. */
int mg_tokenizer_from_text(const char *text, size_t length, uint32_t *characters, size_t capacity, size_t *n);
int mg_tokenizer_encode(const uint32_t *characters, size_t vocab, const char *text, size_t length,
                        uint32_t *tokens, size_t capacity, size_t *n);
int mg_tokenizer_decode(const uint32_t *characters, size_t vocab, const uint32_t *tokens, size_t n, char *out,
                        size_t capacity, size_t *written);

/* Checkpoint (src/gpt/checkpoint.rs:24-192).  mg_checkpoint_load reads the file
 * into a handle; query its parts, then free it. */
typedef struct mg_checkpoint mg_checkpoint;
int mg_checkpoint_load(const char *path, mg_checkpoint **out);
int mg_checkpoint_info(const mg_checkpoint *checkpoint, mg_config *config, size_t *vocab,
                       size_t *parameters);
int mg_checkpoint_characters(const mg_checkpoint *checkpoint, uint32_t *out, size_t n);
int mg_checkpoint_parameters(const mg_checkpoint *checkpoint, float *out, size_t n);
void mg_checkpoint_free(mg_checkpoint *checkpoint);
/* Checkpoint::save (checkpoint.rs:25-94). */
int mg_checkpoint_save(const char *path, const mg_config *config, const uint32_t *characters, size_t vocab,
                       const float *parameters, size_t n);

#ifdef __cplusplus
}
#endif

#endif
