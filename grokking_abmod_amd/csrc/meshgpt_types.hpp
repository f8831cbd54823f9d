// Host-side model types of the Mesh GPT generate path: configuration and its
// validation, the parameter layout and seeded initialisation, fixed token codes,
// the character tokenizer and the weights-only checkpoint format.  These mirror
// the reference's Rust types one for one (names, argument meaning, error text).
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace meshgpt {

// Status codes shared with the C ABI (include/meshgpt.h).
enum Status : int {
    kOk = 0,
    kInvalidArgument = 1,
    kOutOfMemory = 2,
    kDeviceError = 3,
    kNonfinite = 4,
    kIo = 5,
    kUnsupported = 6,
};

// Every failure carries the reference's message text and a C ABI status.
struct Error : std::runtime_error {
    int status;
    explicit Error(const std::string &message, int code = kInvalidArgument)
        : std::runtime_error(message), status(code) {}
};

constexpr uint32_t kIgnoreTarget = 0xFFFFFFFFu;  // IGNORE_TARGET, src/gpt/mod.rs:26
constexpr size_t kMaxRows = 131072;        // src/gpt/mod.rs:31
constexpr size_t kModelMaxWidth = 4096;    // src/gpt/mod.rs:33
constexpr size_t kModelMaxContext = 4096;  // src/gpt/mod.rs:34
constexpr size_t kModelMaxHeads = 64;      // src/gpt/mod.rs:35
constexpr size_t kModelMaxVocab = 65536;   // src/gpt/mod.rs:36
constexpr float kRopeBase = 10000.0f;      // src/gpt/mod.rs:37
constexpr float kRmsEpsilon = 1e-5f;       // src/gpt/mod.rs:38
constexpr float kXsaEpsilon = 1e-12f;      // src/gpt/mod.rs:40
// Long-context extension: contexts beyond 4096 are accepted only when a config
// sets long_context (the reference caps context at 4096, config.rs:148).
constexpr size_t kExtendedMaxContext = 65536;

enum class TokenEmbedding : uint32_t { Mesh = 0, Table = 1 };        // config.rs:58-67
enum class MeshConnectivity : uint32_t { Neighbor = 0, Butterfly = 1 };  // config.rs:96-106

const char *name(TokenEmbedding e);
const char *name(MeshConnectivity c);
TokenEmbedding parse_embedding(const std::string &text);     // config.rs:84-94
MeshConnectivity parse_connectivity(const std::string &text);  // config.rs:131-141

// Distance from a neuron's own channel to its second parent (config.rs:116-122).
size_t stride(MeshConnectivity connectivity, size_t width, size_t layer);

// Token-code geometry ablations (geometry.rs:37-47); the numeric values are
// the checkpoint codes.
enum class EmbeddingForm : uint32_t {
    Parity = 0, Circle, Fourier, Orthogonal, Simplex, Equiangular, Antipodal, Hypercube,
    SignedPermutations, Sphere
};
enum class EmbeddingOrder : uint32_t { Token = 0, Residue, DiscreteLog };
enum class EmbeddingNorm : uint32_t { None = 0, Unit, Rms };

// Their names and parsers (geometry.rs:8-46): "unknown EmbeddingForm: X" etc.
const char *name(EmbeddingForm f);
const char *name(EmbeddingOrder o);
const char *name(EmbeddingNorm n);
EmbeddingForm parse_form(const std::string &text);
EmbeddingOrder parse_order(const std::string &text);
EmbeddingNorm parse_norm(const std::string &text);

// Rust's Display of an f32: the shortest decimal that reads back to the same
// value, never in exponent form.
std::string display_f32(float v);

struct GptConfig;
class CharacterTokenizer;

// EmbeddingGeometry (geometry.rs:49-81); defaults keep the signed parity codes.
// AdamWOptions (config.rs:258-276) with its defaults.
struct AdamWOptions {
    float learning_rate = 0.003f;
    float weight_decay = 0.01f;
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float epsilon = 1e-8f;
    void validate() const;  // config.rs:278-295
};

// GptTrainOptions (config.rs:297-333): the `mesh-gpt train` loop's settings.
struct GptTrainOptions {
    size_t steps = 1000;
    float learning_rate = 0.003f;
    float weight_decay = 0.01f;
    size_t report_every = 100;
    void validate() const;
};

struct EmbeddingGeometry {
    EmbeddingForm form = EmbeddingForm::Parity;
    EmbeddingOrder order = EmbeddingOrder::Token;
    size_t frequency = 1;
    size_t harmonics = 1;
    float overlap = 0.0f;
    EmbeddingNorm normalization = EmbeddingNorm::None;
    bool frozen = false;
    size_t preserve_features = 0;
    size_t modulus = 0;
    uint64_t seed = 0;

    bool operator==(const EmbeddingGeometry &o) const;
    bool is_default() const { return *this == EmbeddingGeometry{}; }
    void validate(const GptConfig &config) const;           // geometry.rs:84-151
    bool transformed() const {                              // geometry.rs:153-155
        return normalization != EmbeddingNorm::None || preserve_features > 0;
    }
    float radius(size_t width) const;                       // geometry.rs:157-162
};

// GptConfig (config.rs:21-56), with the geometry and operator-switch ablations.
struct GptConfig {
    size_t vocab_size = 32;
    size_t context = 32;
    size_t width = 32;
    size_t heads = 4;
    size_t layers = 2;
    size_t attention_mesh_depth = 4;
    size_t ffn_mesh_depth = 6;
    TokenEmbedding embedding = TokenEmbedding::Mesh;
    MeshConnectivity connectivity = MeshConnectivity::Neighbor;
    EmbeddingGeometry geometry;
    bool rope = true;
    bool qk_norm = true;
    bool xsa = true;
    bool long_context = false;  // extension flag, never stored in checkpoints

    bool operator==(const GptConfig &o) const;
    void validate() const;                                                // config.rs:144-172
    size_t parameter_count() const;                                       // config.rs:174-176
    size_t embedding_parameter_count() const;                             // config.rs:179-184
    std::vector<float> initial_parameters(uint64_t seed) const;           // config.rs:187-190
    void validate_tokens(const uint32_t *tokens, size_t n, size_t sequence) const;  // 210-228
    size_t head_width() const { return width / heads; }
    // Every operator on and the default geometry: the MSHGPT07/08 architectures.
    bool reference_operators() const { return rope && qk_norm && xsa && geometry.is_default(); }
};

struct Group {
    size_t offset, size, depth;
};
struct Block {
    size_t query, key, value, projection, ffn;
};

// Layout (config.rs:351-459): the embedding group, then q, k, v, projection and
// ffn meshes of every block; each mesh layer stores [self, partner] per channel.
struct Layout {
    std::vector<Group> groups;
    std::vector<Block> blocks;
    size_t embedding = 0;

    static Layout build(const GptConfig &config);
    size_t count() const;
    std::vector<float> initialize(const GptConfig &config, uint64_t seed) const;
    // Weights drawn from N(0, sigma^2) (BASELINE.json's synthetic workloads;
    // config.rs has no such initialiser): parameter i in flat order (group,
    // layer, channel, self then partner) is sigma times the reference's
    // Box-Muller draw from Random::new(seed) (src/simple/numerical.rs:163-167:
    // two unit() draws, sqrt(-2 ln(1 - u1)) cos(2 pi u2) in f64, rounded to
    // f32), multiplied in f32; protected rows stay zero as in initialize.
    std::vector<float> initialize_normal(const GptConfig &config, uint64_t seed, float sigma) const;
    // The final mesh rows that write protected residual coordinates
    // (config.rs:461-474): [begin, end) within group `id`.
    std::pair<size_t, size_t> constrained_range(const GptConfig &config, size_t id) const;
    // "protected residual output weights must be zero" (config.rs:476-488).
    void validate_constraints(const GptConfig &config, const float *parameters) const;
};

// Fixed token codes, vocab x width (config.rs:552-591; geometric forms and
// orders, geometry.rs:186-325).
std::vector<float> token_codes(const GptConfig &config);
// The residue token permutation of the grok dataset (grokking.rs:260-271).
std::vector<uint32_t> residue_permutation(size_t modulus, uint64_t seed);
// EquationDataset (grokking.rs:116-258): the whole table of a modular
// operation (codes in ModularOperation order: 0 add, 1 multiply, 2 subtract,
// 3 divide, ...), split by a seeded shuffle; batches are a, op, b, '=' with
// only the answer supervised.
struct EquationDataset {
    struct Equation {
        size_t a, b, answer;
    };
    size_t modulus = 0;
    std::vector<Equation> training, validation;
    std::vector<uint32_t> residue_tokens;
    static EquationDataset build(size_t modulus, uint32_t operation, double train_fraction, uint64_t seed);
    // inputs and targets of 4 * n rows for the split's equations `indices`
    void batch(bool validation, const size_t *indices, size_t n, uint32_t *inputs, uint32_t *targets) const;
    // The dataset's tokenizer (grokking.rs:146-157): residue r's token is the
    // private-use character U+E000 + r, then the operation's symbol and '='.
    CharacterTokenizer tokenizer() const;
    uint32_t operation = 0;
};
// TextDataset (text.rs:58-108): a tokenised corpus split 90/10 into training
// and validation; a batch is `batch` windows of `sequence` tokens at seeded
// starts, targets shifted by one.
class TextDataset {
  public:
    TextDataset(const std::vector<uint32_t> &tokens, const GptConfig &config);
    void batch(bool validation, size_t sequence, size_t batch, uint64_t seed, uint32_t *inputs,
               uint32_t *targets) const;
    size_t training_size() const { return training_.size(); }
    size_t validation_size() const { return validation_.size(); }

  private:
    std::vector<uint32_t> training_, validation_;
};
// The smallest primitive root of a prime (geometry.rs:166-184).
size_t primitive_root(size_t prime);
// Table parameters of a mesh-embedding model (config.rs:505-547).
std::vector<float> tabulate_embedding(const GptConfig &config, const std::vector<float> &parameters);

// SplitMix64 (src/mesh.rs:256-288).
class Random {
  public:
    explicit Random(uint64_t seed) : state_(seed) {}
    uint64_t next_u64();
    float unit();
    size_t index(size_t bound);

  private:
    uint64_t state_;
};

// "{name} must contain only finite values" (src/mesh.rs:239-246).
void validate_finite(const float *values, size_t n, const char *name);

// CharacterTokenizer (src/gpt/text.rs:7-56): sorted unique Unicode scalars.
class CharacterTokenizer {
  public:
    static CharacterTokenizer from_text(const std::string &utf8);
    static CharacterTokenizer from_characters(std::vector<uint32_t> characters);
    size_t vocab_size() const { return characters_.size(); }
    std::vector<uint32_t> encode(const std::string &utf8) const;
    std::string decode(const uint32_t *tokens, size_t n) const;
    const std::vector<uint32_t> &characters() const { return characters_; }
    bool operator==(const CharacterTokenizer &o) const { return characters_ == o.characters_; }

  private:
    std::vector<uint32_t> characters_;
};

std::vector<uint32_t> utf8_decode(const std::string &text);
std::string utf8_encode(const uint32_t *scalars, size_t n);

// Weights-only checkpoint (src/gpt/checkpoint.rs:14-201): MSHGPT07 for the
// default architecture, MSHGPT08 with embedding/connectivity codes, MSHGPT09
// with the geometry and operator switches.
struct Checkpoint {
    GptConfig config;
    CharacterTokenizer tokenizer;
    std::vector<float> parameters;

    std::vector<uint8_t> serialize() const;
    void save(const std::string &path) const;
    static Checkpoint read(const uint8_t *bytes, size_t n);
    static Checkpoint load(const std::string &path);
};

}  // namespace meshgpt
