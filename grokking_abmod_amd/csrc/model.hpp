// MeshGpt: the device-resident Mesh GPT used by generate, mirroring the
// reference's SpecializedMeshGpt inference API (src/gpt/gpu.rs:1693-2092) with
// run-time dimensions instead of compile-time capacities, a KV cache, batched
// sequences and on-device sampling.
#pragma once

#include <hip/hip_runtime_api.h>

#include <memory>
#include <string>
#include <vector>

#include "meshgpt_types.hpp"

namespace meshgpt {

class MeshGpt {
  public:
    // gpu.rs:1718-1771: validates the config, seeds the weights with `seed` and
    // keeps decode state for up to max_batch sequences (grown on demand).
    MeshGpt(int device, const GptConfig &config, uint64_t seed, size_t max_batch = 1);
    ~MeshGpt();
    MeshGpt(const MeshGpt &) = delete;
    MeshGpt &operator=(const MeshGpt &) = delete;

    const GptConfig &config() const;
    std::vector<float> parameters() const;                  // gpu.rs:1846-1853
    void set_parameters(const float *values, size_t n);     // gpu.rs:1856-1872
    // gpu.rs:1875-1887: logits of every row (or only each sequence's last row)
    std::vector<float> logits(const uint32_t *tokens, size_t n, size_t sequence, bool last_only = false);
    std::vector<float> token_embeddings();                  // gpu.rs:2056-2068, V x W
    std::vector<float> hidden_states(const uint32_t *tokens, size_t n, size_t sequence);  // gpu.rs:2070
    // Training (gpu.rs:1915-2003).  Targets equal to kIgnoreTarget are not
    // supervised.  cross_entropy: the mean next-token loss; loss_and_gradient:
    // the loss and the gradient of every parameter (masked as config.rs:490-500);
    // train_batch: the loss before one AdamW update of the weights (the moments
    // persist across calls until set_parameters).
    double cross_entropy(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence);
    double loss_and_gradient(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                             std::vector<float> &gradient);
    double train_batch(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                       const AdamWOptions &options);
    // Bytes of device memory the model holds (gpu.rs allocated_device_bytes).
    size_t allocated_device_bytes() const;
    // gpu.rs:2006-2053 on text; batch rows b use seed + b.
    std::string generate(const CharacterTokenizer &tokenizer, const std::string &prompt, size_t count,
                         float temperature, uint64_t seed);
    // Token-level batched generate: prompts[B][P] -> out[B][P+count].
    void generate_tokens(const uint32_t *prompts, size_t batch, size_t prompt_len, size_t count,
                         float temperature, uint64_t seed, uint32_t *out);

    // Step-wise decode surface used by the benchmark: prefill samples the first
    // token; decode(k) runs k more on-device steps (KV path only).
    void prefill(const uint32_t *prompts, size_t batch, size_t prompt_len, float temperature,
                 uint64_t seed, size_t reserve);
    void decode(size_t steps);
    // Back to the state the last prefill() left (lengths and sampler states).
    void rewind();
    // Kernel time (ms, HIP events) of the last logits / hidden_states / prefill call.
    float last_call_ms() const;
    // Same steps without graph replay, timing every decode-attention launch
    // with HIP events; returns milliseconds per launch (steps x layers).
    std::vector<float> decode_profiled(size_t steps);
    // Same steps in one persistent launch that records its timeline: blocks x
    // steps x (layers + 1) x 2 wall-clock stamps (100 MHz), layout as
    // kern::PersistArgs::trace; blocks are 3*batch mesh teams then
    // batch*heads attention blocks.
    std::vector<uint64_t> decode_traced(size_t steps);
    size_t sequence_length() const;
    void read_tokens(uint32_t *out, size_t batch, size_t length);
    std::vector<float> last_logits();
    hipStream_t stream() const;
    void synchronize();

  private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// The generate sampler on device for `rows` rows of `vocab` logits: greedy
// when temperature == 0, else one draw from rng_states[r] per row (advanced in
// place).  Returns whether any row held a non-finite logit.
bool sample_logits(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                   uint64_t *rng_states, uint32_t *tokens);
// sample_logits on device-resident buffers, enqueued on `stream` without
// waiting or allocating: its only scratch is the fixed per-device array of
// kern::kNoAllocRows row counters.  *nonfinite (device) receives 1 when a row
// holds a non-finite logit, else 0.
void sample_logits_noalloc(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                           uint64_t *rng_states, uint32_t *tokens, int *nonfinite, hipStream_t stream);
// out[i] = the sampler's f32 exp of x[i], evaluated on `device`.
void device_expf(int device, const float *x, size_t n, float *out);

// Mean bandwidth (read + write bytes / s / 1e9) of a plain device copy of
// `bytes`, repeated `iters` times on `device`.
double copy_bandwidth(int device, size_t bytes, int iters);

}  // namespace meshgpt
