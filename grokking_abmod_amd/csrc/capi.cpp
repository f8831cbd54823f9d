// extern "C" surface of include/meshgpt.h over the C++ model types.
#include "../../include/meshgpt.h"

#include <cstring>
#include <new>
#include <string>

#include "meshgpt_types.hpp"
#include "model.hpp"

using namespace meshgpt;

struct mg_model {
    MeshGpt model;
    mg_model(int device, const GptConfig &config, uint64_t seed, size_t max_batch)
        : model(device, config, seed, max_batch) {}
};

struct mg_checkpoint {
    Checkpoint checkpoint;
};

namespace {

thread_local std::string last_error;

template <class F>
int guarded(F &&f) {
    try {
        f();
        last_error.clear();
        return MG_OK;
    } catch (const Error &e) {
        last_error = e.what();
        return e.status;
    } catch (const std::bad_alloc &) {
        last_error = "out of host memory";
        return MG_OUT_OF_MEMORY;
    } catch (const std::exception &e) {
        last_error = e.what();
        return MG_INVALID_ARGUMENT;
    }
}

void require(bool ok, const char *message) {
    if (!ok) throw Error(message);
}

GptConfig to_config(const mg_config *c) {
    require(c != nullptr, "config must not be null");
    GptConfig g;
    g.vocab_size = c->vocab_size;
    g.context = c->context;
    g.width = c->width;
    g.heads = c->heads;
    g.layers = c->layers;
    g.attention_mesh_depth = c->attention_mesh_depth;
    g.ffn_mesh_depth = c->ffn_mesh_depth;
    require(c->embedding <= 1, "unknown token embedding code");
    require(c->connectivity <= 1, "unknown mesh connectivity code");
    g.embedding = TokenEmbedding(c->embedding);
    g.connectivity = MeshConnectivity(c->connectivity);
    g.long_context = c->long_context != 0;
    require(c->rope <= 1 && c->qk_norm <= 1 && c->xsa <= 1 && c->frozen <= 1, "invalid checkpoint switch");
    g.rope = c->rope != 0;
    g.qk_norm = c->qk_norm != 0;
    g.xsa = c->xsa != 0;
    if (c->form > 9) throw Error("unknown checkpoint EmbeddingForm: " + std::to_string(c->form));
    if (c->order > 2) throw Error("unknown checkpoint EmbeddingOrder: " + std::to_string(c->order));
    if (c->normalization > 2)
        throw Error("unknown checkpoint EmbeddingNorm: " + std::to_string(c->normalization));
    g.geometry.form = EmbeddingForm(c->form);
    g.geometry.order = EmbeddingOrder(c->order);
    g.geometry.frequency = c->frequency;
    g.geometry.harmonics = c->harmonics;
    g.geometry.overlap = c->overlap;
    g.geometry.normalization = EmbeddingNorm(c->normalization);
    g.geometry.frozen = c->frozen != 0;
    g.geometry.preserve_features = c->preserve_features;
    g.geometry.modulus = c->modulus;
    g.geometry.seed = c->seed;
    return g;
}

void from_config(const GptConfig &g, mg_config *c) {
    c->vocab_size = uint32_t(g.vocab_size);
    c->context = uint32_t(g.context);
    c->width = uint32_t(g.width);
    c->heads = uint32_t(g.heads);
    c->layers = uint32_t(g.layers);
    c->attention_mesh_depth = uint32_t(g.attention_mesh_depth);
    c->ffn_mesh_depth = uint32_t(g.ffn_mesh_depth);
    c->embedding = uint32_t(g.embedding);
    c->connectivity = uint32_t(g.connectivity);
    c->long_context = g.long_context ? 1 : 0;
    c->rope = g.rope;
    c->qk_norm = g.qk_norm;
    c->xsa = g.xsa;
    c->form = uint32_t(g.geometry.form);
    c->order = uint32_t(g.geometry.order);
    c->frequency = uint32_t(g.geometry.frequency);
    c->harmonics = uint32_t(g.geometry.harmonics);
    c->overlap = g.geometry.overlap;
    c->normalization = uint32_t(g.geometry.normalization);
    c->frozen = g.geometry.frozen;
    c->preserve_features = uint32_t(g.geometry.preserve_features);
    c->modulus = uint32_t(g.geometry.modulus);
    c->seed = g.geometry.seed;
}

MeshGpt &model_of(mg_model *m) {
    require(m != nullptr, "model must not be null");
    return m->model;
}

void copy_out(const std::vector<float> &v, float *out, size_t n) {
    require(out != nullptr && n >= v.size(), "output buffer is too small");
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

}  // namespace

extern "C" {

const char *mg_last_error(void) { return last_error.c_str(); }

void mg_config_default(mg_config *out) {
    if (out) from_config(GptConfig{}, out);
}

int mg_config_validate(const mg_config *config) {
    return guarded([&] { to_config(config).validate(); });
}

int mg_parameter_count(const mg_config *config, size_t *out) {
    return guarded([&] {
        require(out != nullptr, "output must not be null");
        *out = to_config(config).parameter_count();
    });
}

int mg_initial_parameters(const mg_config *config, uint64_t seed, float *out, size_t n) {
    return guarded([&] { copy_out(to_config(config).initial_parameters(seed), out, n); });
}

int mg_normal_parameters(const mg_config *config, uint64_t seed, float sigma, float *out, size_t n) {
    return guarded([&] {
        GptConfig g = to_config(config);
        g.validate();
        copy_out(Layout::build(g).initialize_normal(g, seed, sigma), out, n);
    });
}

int mg_token_codes(const mg_config *config, float *out, size_t n) {
    return guarded([&] {
        GptConfig g = to_config(config);
        g.validate();
        copy_out(token_codes(g), out, n);
    });
}

int mg_model_create(int device, const mg_config *config, uint64_t seed, size_t max_batch, mg_model **out) {
    return guarded([&] {
        require(out != nullptr, "output must not be null");
        *out = nullptr;
        *out = new mg_model(device, to_config(config), seed, max_batch);
    });
}

void mg_model_destroy(mg_model *model) { delete model; }

int mg_model_config(const mg_model *model, mg_config *out) {
    return guarded([&] {
        require(model != nullptr && out != nullptr, "model and output must not be null");
        from_config(model->model.config(), out);
    });
}

int mg_parameters(mg_model *model, float *out, size_t n) {
    return guarded([&] { copy_out(model_of(model).parameters(), out, n); });
}

int mg_set_parameters(mg_model *model, const float *values, size_t n) {
    return guarded([&] {
        require(values != nullptr || n == 0, "parameters must not be null");
        model_of(model).set_parameters(values, n);
    });
}

int mg_logits(mg_model *model, const uint32_t *tokens, size_t n, size_t sequence, int last_only, float *out,
              size_t out_len) {
    return guarded([&] {
        require(tokens != nullptr || n == 0, "tokens must not be null");
        static const uint32_t none = 0;
        copy_out(model_of(model).logits(tokens ? tokens : &none, n, sequence, last_only != 0), out, out_len);
    });
}

int mg_equation_split(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed, size_t *n_train,
                      size_t *n_valid) {
    return guarded([&] {
        require(n_train != nullptr && n_valid != nullptr, "outputs must not be null");
        const EquationDataset d = EquationDataset::build(modulus, operation, train_fraction, seed);
        *n_train = d.training.size();
        *n_valid = d.validation.size();
    });
}

int mg_equation_batch(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed, int validation,
                      const size_t *indices, size_t n, uint32_t *inputs, uint32_t *targets) {
    return guarded([&] {
        require((indices != nullptr || n == 0) && inputs != nullptr && targets != nullptr,
                "indices and outputs must not be null");
        EquationDataset::build(modulus, operation, train_fraction, seed)
            .batch(validation != 0, indices, n, inputs, targets);
    });
}

int mg_text_batch(const uint32_t *tokens, size_t n_tokens, const mg_config *config, int validation,
                  size_t sequence, size_t batch, uint64_t seed, uint32_t *inputs, uint32_t *targets) {
    return guarded([&] {
        require((tokens != nullptr || n_tokens == 0) && inputs != nullptr && targets != nullptr,
                "tokens and outputs must not be null");
        const TextDataset d(std::vector<uint32_t>(tokens, tokens + n_tokens), to_config(config));
        d.batch(validation != 0, sequence, batch, seed, inputs, targets);
    });
}

void mg_adamw_default(mg_adamw *out) {
    if (!out) return;
    const AdamWOptions d;
    *out = mg_adamw{d.learning_rate, d.weight_decay, d.beta1, d.beta2, d.epsilon};
}

int mg_cross_entropy(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                     double *loss) {
    return guarded([&] {
        require(inputs != nullptr && targets != nullptr && loss != nullptr, "inputs, targets and loss must not be null");
        *loss = model_of(model).cross_entropy(inputs, targets, n, sequence);
    });
}

int mg_loss_and_gradient(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n,
                         size_t sequence, double *loss, float *gradient, size_t n_gradient) {
    return guarded([&] {
        require(inputs != nullptr && targets != nullptr && loss != nullptr, "inputs, targets and loss must not be null");
        std::vector<float> g;
        const double l = model_of(model).loss_and_gradient(inputs, targets, n, sequence, g);
        copy_out(g, gradient, n_gradient);
        *loss = l;
    });
}

int mg_train_batch(mg_model *model, const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                   const mg_adamw *options, double *loss) {
    return guarded([&] {
        require(inputs != nullptr && targets != nullptr && options != nullptr && loss != nullptr,
                "inputs, targets, options and loss must not be null");
        AdamWOptions o;
        o.learning_rate = options->learning_rate;
        o.weight_decay = options->weight_decay;
        o.beta1 = options->beta1;
        o.beta2 = options->beta2;
        o.epsilon = options->epsilon;
        *loss = model_of(model).train_batch(inputs, targets, n, sequence, o);
    });
}

int mg_token_embeddings(mg_model *model, float *out, size_t n) {
    return guarded([&] { copy_out(model_of(model).token_embeddings(), out, n); });
}

int mg_hidden_states(mg_model *model, const uint32_t *tokens, size_t n, size_t sequence, float *out,
                     size_t out_len) {
    return guarded([&] {
        require(tokens != nullptr || n == 0, "tokens must not be null");
        static const uint32_t none = 0;
        copy_out(model_of(model).hidden_states(tokens ? tokens : &none, n, sequence), out, out_len);
    });
}

int mg_generate(mg_model *model, const uint32_t *prompts, size_t batch, size_t prompt_len, size_t count,
                float temperature, uint64_t seed, uint32_t *out) {
    return guarded([&] {
        require((prompts != nullptr || batch * prompt_len == 0) && out != nullptr,
                "prompts and output must not be null");
        model_of(model).generate_tokens(prompts, batch, prompt_len, count, temperature, seed, out);
    });
}

int mg_generate_text(mg_model *model, const uint32_t *characters, size_t vocab, const char *prompt,
                     size_t count, float temperature, uint64_t seed, char *out, size_t capacity,
                     size_t *written) {
    return guarded([&] {
        require(characters != nullptr && prompt != nullptr && written != nullptr,
                "characters, prompt and length must not be null");
        CharacterTokenizer tokenizer =
            CharacterTokenizer::from_characters(std::vector<uint32_t>(characters, characters + vocab));
        std::string text = model_of(model).generate(tokenizer, prompt, count, temperature, seed);
        *written = text.size();
        require(out != nullptr && capacity >= text.size(), "output buffer is too small");
        std::memcpy(out, text.data(), text.size());
    });
}

int mg_prefill(mg_model *model, const uint32_t *prompts, size_t batch, size_t prompt_len, float temperature,
               uint64_t seed, size_t reserve) {
    return guarded([&] {
        require(prompts != nullptr, "prompts must not be null");
        model_of(model).prefill(prompts, batch, prompt_len, temperature, seed, reserve);
    });
}

int mg_decode(mg_model *model, size_t steps) {
    return guarded([&] { model_of(model).decode(steps); });
}

int mg_last_call_ms(mg_model *model, float *ms) {
    return guarded([&] {
        require(ms != nullptr, "output must not be null");
        *ms = model_of(model).last_call_ms();
    });
}

int mg_decode_rewind(mg_model *model) {
    return guarded([&] { model_of(model).rewind(); });
}

int mg_decode_profiled(mg_model *model, size_t steps, float *ms, size_t n) {
    return guarded([&] { copy_out(model_of(model).decode_profiled(steps), ms, n); });
}

int mg_decode_traced(mg_model *model, size_t steps, uint64_t *stamps, size_t n) {
    return guarded([&] {
        const std::vector<uint64_t> t = model_of(model).decode_traced(steps);
        require(stamps != nullptr && n >= t.size(), "output buffer is too small");
        std::memcpy(stamps, t.data(), t.size() * 8);
    });
}

int mg_sequence_length(const mg_model *model, size_t *out) {
    return guarded([&] {
        require(model != nullptr && out != nullptr, "model and output must not be null");
        *out = model->model.sequence_length();
    });
}

int mg_read_tokens(mg_model *model, uint32_t *out, size_t batch, size_t length) {
    return guarded([&] {
        require(out != nullptr, "output must not be null");
        model_of(model).read_tokens(out, batch, length);
    });
}

int mg_last_logits(mg_model *model, float *out, size_t n) {
    return guarded([&] { copy_out(model_of(model).last_logits(), out, n); });
}

void *mg_model_stream(mg_model *model) { return model ? static_cast<void *>(model->model.stream()) : nullptr; }

int mg_sample_logits(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                     uint64_t *rng_states, uint32_t *tokens) {
    return guarded([&] {
        require((logits != nullptr && rng_states != nullptr && tokens != nullptr) || rows == 0,
                "logits, states and tokens must not be null");
        if (sample_logits(device, logits, rows, vocab, temperature, rng_states, tokens))
            throw Error("logits must contain only finite values", kNonfinite);
    });
}

int mg_sample_logits_noalloc(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                             uint64_t *rng_states, uint32_t *tokens, int *nonfinite, void *stream) {
    return guarded([&] {
        require((logits != nullptr && rng_states != nullptr && tokens != nullptr) || rows == 0,
                "logits, states and tokens must not be null");
        sample_logits_noalloc(device, logits, rows, vocab, temperature, rng_states, tokens, nonfinite,
                              static_cast<hipStream_t>(stream));
    });
}

int mg_expf(int device, const float *x, size_t n, float *out) {
    return guarded([&] {
        require((x != nullptr && out != nullptr) || n == 0, "inputs and outputs must not be null");
        device_expf(device, x, n, out);
    });
}

int mg_copy_bandwidth(int device, size_t bytes, int iters, double *gbps) {
    return guarded([&] {
        require(gbps != nullptr && bytes >= 16 && iters >= 1, "bytes >= 16, iters >= 1 and output required");
        *gbps = copy_bandwidth(device, bytes, iters);
    });
}

int mg_tokenizer_from_text(const char *text, size_t length, uint32_t *characters, size_t capacity, size_t *n) {
    return guarded([&] {
        require(text != nullptr || length == 0, "text must not be null");
        require(n != nullptr, "output must not be null");
        const auto t = CharacterTokenizer::from_text(std::string(text ? text : "", length));
        *n = t.vocab_size();
        if (characters) {
            require(capacity >= t.vocab_size(), "output buffer is too small");
            std::memcpy(characters, t.characters().data(), t.vocab_size() * 4);
        }
    });
}

int mg_tokenizer_encode(const uint32_t *characters, size_t vocab, const char *text, size_t length,
                        uint32_t *tokens, size_t capacity, size_t *n) {
    return guarded([&] {
        require(characters != nullptr && (text != nullptr || length == 0) && n != nullptr,
                "characters, text and output must not be null");
        const auto t = CharacterTokenizer::from_characters(std::vector<uint32_t>(characters, characters + vocab));
        const auto ids = t.encode(std::string(text ? text : "", length));
        require(tokens != nullptr || ids.empty(), "output must not be null");
        require(capacity >= ids.size(), "output buffer is too small");
        if (!ids.empty()) std::memcpy(tokens, ids.data(), ids.size() * 4);
        *n = ids.size();
    });
}

int mg_tokenizer_decode(const uint32_t *characters, size_t vocab, const uint32_t *tokens, size_t n, char *out,
                        size_t capacity, size_t *written) {
    return guarded([&] {
        require(characters != nullptr && (tokens != nullptr || n == 0) && written != nullptr,
                "characters, tokens and output must not be null");
        const auto t = CharacterTokenizer::from_characters(std::vector<uint32_t>(characters, characters + vocab));
        const std::string text = t.decode(tokens, n);
        require(out != nullptr || text.empty(), "output must not be null");
        require(capacity >= text.size(), "output buffer is too small");
        if (!text.empty()) std::memcpy(out, text.data(), text.size());
        *written = text.size();
    });
}

int mg_checkpoint_load(const char *path, mg_checkpoint **out) {
    return guarded([&] {
        require(path != nullptr && out != nullptr, "path and output must not be null");
        *out = nullptr;
        *out = new mg_checkpoint{Checkpoint::load(path)};
    });
}

int mg_checkpoint_info(const mg_checkpoint *checkpoint, mg_config *config, size_t *vocab, size_t *parameters) {
    return guarded([&] {
        require(checkpoint != nullptr, "checkpoint must not be null");
        if (config) from_config(checkpoint->checkpoint.config, config);
        if (vocab) *vocab = checkpoint->checkpoint.tokenizer.vocab_size();
        if (parameters) *parameters = checkpoint->checkpoint.parameters.size();
    });
}

int mg_checkpoint_characters(const mg_checkpoint *checkpoint, uint32_t *out, size_t n) {
    return guarded([&] {
        require(checkpoint != nullptr, "checkpoint must not be null");
        const auto &c = checkpoint->checkpoint.tokenizer.characters();
        require(out != nullptr && n >= c.size(), "output buffer is too small");
        std::memcpy(out, c.data(), c.size() * 4);
    });
}

int mg_checkpoint_parameters(const mg_checkpoint *checkpoint, float *out, size_t n) {
    return guarded([&] {
        require(checkpoint != nullptr, "checkpoint must not be null");
        copy_out(checkpoint->checkpoint.parameters, out, n);
    });
}

void mg_checkpoint_free(mg_checkpoint *checkpoint) { delete checkpoint; }

int mg_checkpoint_save(const char *path, const mg_config *config, const uint32_t *characters, size_t vocab,
                       const float *parameters, size_t n) {
    return guarded([&] {
        require(path != nullptr && characters != nullptr && (parameters != nullptr || n == 0),
                "path, characters and parameters must not be null");
        Checkpoint ck;
        ck.config = to_config(config);
        ck.tokenizer = CharacterTokenizer::from_characters(std::vector<uint32_t>(characters, characters + vocab));
        ck.parameters.assign(parameters, parameters + n);
        ck.save(path);
    });
}

}  // extern "C"
