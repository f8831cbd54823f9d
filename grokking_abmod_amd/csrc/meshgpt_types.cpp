// Host-side model types.  Compiled without floating-point contraction: the
// reference's Rust never fuses multiply-add pairs, and the seeded f32
// initialisation below must be bit-identical to it.
#include "meshgpt_types.hpp"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <set>

namespace meshgpt {

const char *name(TokenEmbedding e) { return e == TokenEmbedding::Mesh ? "mesh" : "table"; }
const char *name(MeshConnectivity c) {
    return c == MeshConnectivity::Neighbor ? "neighbor" : "butterfly";
}

TokenEmbedding parse_embedding(const std::string &text) {
    if (text == "mesh") return TokenEmbedding::Mesh;
    if (text == "table") return TokenEmbedding::Table;
    throw Error("unknown token embedding: " + text);
}

MeshConnectivity parse_connectivity(const std::string &text) {
    if (text == "neighbor") return MeshConnectivity::Neighbor;
    if (text == "butterfly") return MeshConnectivity::Butterfly;
    throw Error("unknown mesh connectivity: " + text);
}

namespace {
const char *const kFormNames[] = {"parity",     "circle",    "fourier",   "orthogonal",          "simplex",
                                  "equiangular", "antipodal", "hypercube", "signed-permutations", "sphere"};
const char *const kOrderNames[] = {"token", "residue", "discrete-log"};
const char *const kNormNames[] = {"none", "unit", "rms"};

template <class E, size_t N>
E parse_named(const char *const (&names)[N], const std::string &text, const char *type) {
    for (size_t i = 0; i < N; ++i)
        if (text == names[i]) return E(i);
    throw Error(std::string("unknown ") + type + ": " + text);
}
}  // namespace

const char *name(EmbeddingForm f) { return kFormNames[uint32_t(f)]; }
const char *name(EmbeddingOrder o) { return kOrderNames[uint32_t(o)]; }
const char *name(EmbeddingNorm n) { return kNormNames[uint32_t(n)]; }
EmbeddingForm parse_form(const std::string &t) { return parse_named<EmbeddingForm>(kFormNames, t, "EmbeddingForm"); }
EmbeddingOrder parse_order(const std::string &t) {
    return parse_named<EmbeddingOrder>(kOrderNames, t, "EmbeddingOrder");
}
EmbeddingNorm parse_norm(const std::string &t) { return parse_named<EmbeddingNorm>(kNormNames, t, "EmbeddingNorm"); }

std::string display_f32(float v) {
    if (std::isnan(v)) return "NaN";
    if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
    char buf[96];
    auto res = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::fixed);
    return std::string(buf, res.ptr);
}

static size_t ilog2(size_t x) {
    size_t r = 0;
    while (x >>= 1) ++r;
    return r;
}

size_t stride(MeshConnectivity connectivity, size_t width, size_t layer) {
    if (connectivity == MeshConnectivity::Neighbor) return 1;
    return size_t(1) << (layer % ilog2(width));
}

bool GptConfig::operator==(const GptConfig &o) const {
    return vocab_size == o.vocab_size && context == o.context && width == o.width &&
           heads == o.heads && layers == o.layers &&
           attention_mesh_depth == o.attention_mesh_depth && ffn_mesh_depth == o.ffn_mesh_depth &&
           embedding == o.embedding && connectivity == o.connectivity && geometry == o.geometry &&
           rope == o.rope && qk_norm == o.qk_norm && xsa == o.xsa && long_context == o.long_context;
}

void GptConfig::validate() const {
    if (vocab_size < 2 || vocab_size > kModelMaxVocab) throw Error("vocab_size must be in 2..65536");
    size_t max_context = long_context ? kExtendedMaxContext : kModelMaxContext;
    if (context < 1 || context > max_context)
        throw Error(long_context ? "context must be in 1..65536" : "context must be in 1..4096");
    if (width < 2 || width > kModelMaxWidth) throw Error("width must be in 2..4096");
    if (heads < 1 || heads > kModelMaxHeads || width % heads != 0)
        throw Error("heads must be in 1..64 and divide width");
    if (width / heads < 2) throw Error("each attention head requires at least two channels");
    if (rope && (width / heads) % 2 != 0)
        throw Error("slice RoPE requires an even number of channels per head");
    if (layers < 1 || layers > 64) throw Error("layers must be in 1..64");
    if (attention_mesh_depth < 1 || attention_mesh_depth > 256 || ffn_mesh_depth < 1 ||
        ffn_mesh_depth > 256)
        throw Error("mesh depths must be in 1..256");
    geometry.validate(*this);
}

size_t GptConfig::embedding_parameter_count() const {
    return embedding == TokenEmbedding::Mesh ? 2 * width * attention_mesh_depth
                                             : vocab_size * width;
}

size_t GptConfig::parameter_count() const { return Layout::build(*this).count(); }

std::vector<float> GptConfig::initial_parameters(uint64_t seed) const {
    return Layout::build(*this).initialize(*this, seed);
}

void AdamWOptions::validate() const {
    auto fin = [](float x) { return std::isfinite(x); };
    if (!fin(learning_rate) || learning_rate <= 0.0f || !fin(weight_decay) || weight_decay < 0.0f || !fin(beta1) ||
        !(beta1 >= 0.0f && beta1 < 1.0f) || !fin(beta2) || !(beta2 >= 0.0f && beta2 < 1.0f) || !fin(epsilon) ||
        epsilon <= 0.0f)
        throw Error("AdamW requires finite positive learning rate/epsilon, nonnegative decay, and betas in [0, 1)");
}

void GptTrainOptions::validate() const {
    if (steps == 0 || report_every == 0) throw Error("steps and report_every must be positive");
    if (!std::isfinite(learning_rate) || learning_rate <= 0.0f || !std::isfinite(weight_decay) || weight_decay < 0.0f)
        throw Error("learning_rate must be positive and weight_decay nonnegative; both must be finite");
}

TextDataset::TextDataset(const std::vector<uint32_t> &tokens, const GptConfig &config) {
    config.validate();
    for (uint32_t id : tokens)
        if (id >= config.vocab_size) throw Error("dataset has invalid token IDs");
    const size_t split = tokens.size() * 9 / 10;
    if (split <= config.context || tokens.size() - split <= config.context)
        throw Error("corpus is too short for a 90/10 split at this context length");
    training_.assign(tokens.begin(), tokens.begin() + split);
    validation_.assign(tokens.begin() + split, tokens.end());
}

void TextDataset::batch(bool validation, size_t sequence, size_t batch, uint64_t seed, uint32_t *inputs,
                        uint32_t *targets) const {
    const std::vector<uint32_t> &corpus = validation ? validation_ : training_;
    if (sequence == 0 || sequence >= corpus.size() || batch == 0 || batch > kMaxRows / sequence)
        throw Error("invalid dataset batch dimensions");
    Random random(seed);
    for (size_t b = 0; b < batch; ++b) {
        // An f32 product truncated toward zero, as the reference's `as usize`.
        // Beyond 2^24 windows the product can round up to the last start,
        // whose target would lie past the corpus (the reference's slice
        // panics there); that is an error here.
        const size_t start = size_t(random.unit() * float(corpus.size() - sequence));
        if (start + sequence >= corpus.size()) throw Error("invalid dataset batch dimensions");
        std::copy_n(corpus.begin() + start, sequence, inputs + b * sequence);
        std::copy_n(corpus.begin() + start + 1, sequence, targets + b * sequence);
    }
}

void GptConfig::validate_tokens(const uint32_t *tokens, size_t n, size_t sequence) const {
    if (sequence == 0 || sequence > context || n == 0 || n % sequence != 0 || n > kMaxRows)
        throw Error(
            "tokens must form a nonempty batch of equal sequences within context and 131072 rows");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= vocab_size) throw Error("token ID is outside the vocabulary");
}

Layout Layout::build(const GptConfig &config) {
    config.validate();
    Layout layout;
    auto push = [&layout](size_t size, size_t depth) {
        size_t id = layout.groups.size();
        layout.groups.push_back(Group{layout.count(), size, depth});
        return id;
    };
    layout.embedding = push(config.embedding_parameter_count(),
                            config.embedding == TokenEmbedding::Mesh ? config.attention_mesh_depth : 0);
    size_t mesh = 2 * config.width * config.attention_mesh_depth;
    for (size_t b = 0; b < config.layers; ++b) {
        Block block{};
        block.query = push(mesh, config.attention_mesh_depth);
        block.key = push(mesh, config.attention_mesh_depth);
        block.value = push(mesh, config.attention_mesh_depth);
        block.projection = push(mesh, config.attention_mesh_depth);
        block.ffn = push(2 * config.width * config.ffn_mesh_depth, config.ffn_mesh_depth);
        layout.blocks.push_back(block);
    }
    return layout;
}

size_t Layout::count() const { return groups.empty() ? 0 : groups.back().offset + groups.back().size; }

std::vector<float> Layout::initialize(const GptConfig &config, uint64_t seed) const {
    if (config.embedding == TokenEmbedding::Table) {
        // The table starts as the vectors the seeded embedding mesh generates
        // (config.rs:416-435), so mesh and table models begin as one function;
        // a geometric form's table starts as its codes.
        GptConfig mesh = config;
        mesh.embedding = TokenEmbedding::Mesh;
        Layout layout = Layout::build(mesh);
        std::vector<float> parameters = tabulate_embedding(mesh, layout.initialize(mesh, seed));
        if (config.geometry.form != EmbeddingForm::Parity) {
            const std::vector<float> codes = token_codes(config);
            std::copy(codes.begin(), codes.end(), parameters.begin());
        }
        return parameters;
    }
    Random random(seed);
    std::vector<float> parameters(count(), 0.0f);
    for (const Group &group : groups) {
        float *values = parameters.data() + group.offset;
        for (size_t layer = 0; layer < group.depth; ++layer) {
            for (size_t channel = 0; channel < config.width; ++channel) {
                size_t offset = layer * 2 * config.width + channel * 2;
                float u0 = random.unit();
                float spread = 0.2f * (u0 - 0.5f);
                values[offset] = 0.7f + spread;
                float u1 = random.unit();
                values[offset + 1] = 0.4f * (u1 - 0.5f);
                if (layer + 1 == group.depth) {
                    values[offset] *= 0.3f;
                    values[offset + 1] *= 0.3f;
                }
            }
        }
    }
    for (size_t id = 0; id < groups.size(); ++id) {
        const auto [begin, end] = constrained_range(config, id);
        std::fill(parameters.begin() + groups[id].offset + begin, parameters.begin() + groups[id].offset + end,
                  0.0f);
    }
    return parameters;
}

std::vector<float> Layout::initialize_normal(const GptConfig &config, uint64_t seed, float sigma) const {
    if (!std::isfinite(sigma) || sigma < 0.0f) throw Error("normal initialisation needs a finite nonnegative sigma");
    Random random(seed);
    std::vector<float> parameters(count());
    for (float &value : parameters) {
        const double u1 = double(random.unit()), u2 = double(random.unit());
        const double radius = std::sqrt(-2.0 * std::log(1.0 - u1));
        const double angle = 6.283185307179586 * u2;  // f64 TAU
        value = float(radius * std::cos(angle)) * sigma;
    }
    for (size_t id = 0; id < groups.size(); ++id) {
        const auto [begin, end] = constrained_range(config, id);
        std::fill(parameters.begin() + groups[id].offset + begin, parameters.begin() + groups[id].offset + end,
                  0.0f);
    }
    return parameters;
}

std::pair<size_t, size_t> Layout::constrained_range(const GptConfig &config, size_t id) const {
    if (config.geometry.preserve_features == 0) return {0, 0};
    for (const Block &b : blocks)
        if (b.projection == id || b.ffn == id) {
            const size_t begin = groups[id].size - 2 * config.width;
            return {begin, begin + 2 * config.geometry.preserve_features};
        }
    return {0, 0};
}

void Layout::validate_constraints(const GptConfig &config, const float *parameters) const {
    for (size_t id = 0; id < groups.size(); ++id) {
        const auto [begin, end] = constrained_range(config, id);
        for (size_t i = groups[id].offset + begin; i < groups[id].offset + end; ++i)
            if (parameters[i] != 0.0f) throw Error("protected residual output weights must be zero");
    }
}

std::vector<float> geometric_codes(const GptConfig &config);
std::vector<float> reorder_parity(const GptConfig &config, const std::vector<float> &codes);

std::vector<float> token_codes(const GptConfig &config) {
    if (config.geometry.form != EmbeddingForm::Parity) return geometric_codes(config);
    const size_t V = config.vocab_size, W = config.width;
    size_t bits = 0;
    for (size_t v = V - 1; v; v >>= 1) ++bits;
    size_t lanes = std::min(W, bits);
    // Single bits first keep codes injective; non-power-of-two masks add parities.
    std::vector<size_t> masks;
    for (size_t b = 0; b < bits; ++b) masks.push_back(size_t(1) << b);
    for (size_t m = 1; m < (size_t(1) << bits); ++m)
        if (m & (m - 1)) masks.push_back(m);
    std::vector<float> codes(V * W);
    for (size_t token = 0; token < V; ++token) {
        for (size_t channel = 0; channel < W; ++channel) {
            float value;
            if (W >= bits) {
                value = (__builtin_popcountll(token & masks[channel % masks.size()]) % 2 == 0) ? -1.0f
                                                                                              : 1.0f;
            } else {
                // Narrow widths pack disjoint bit groups into signed radix digits.
                uint64_t digit = 0, maximum = 0;
                for (size_t bit = channel % lanes; bit < bits; bit += lanes) {
                    digit = 2 * digit + ((token >> bit) & 1);
                    maximum = 2 * maximum + 1;
                }
                value = 2.0f * float(digit) / float(maximum) - 1.0f;
            }
            codes[token * W + channel] = value;
        }
    }
    return reorder_parity(config, codes);
}

std::vector<float> tabulate_embedding(const GptConfig &config, const std::vector<float> &parameters) {
    if (config.embedding != TokenEmbedding::Mesh || parameters.size() != config.parameter_count())
        throw Error("tabulation requires the parameters of a mesh-embedding configuration");
    validate_finite(parameters.data(), parameters.size(), "parameters");
    const size_t V = config.vocab_size, W = config.width, depth = config.attention_mesh_depth;
    std::vector<float> codes = token_codes(config);
    std::vector<double> vec(codes.begin(), codes.end()), input(W);
    for (size_t layer = 0; layer < depth; ++layer) {
        size_t s = stride(config.connectivity, W, layer);
        for (size_t t = 0; t < V; ++t) {
            double *v = vec.data() + t * W;
            std::copy(v, v + W, input.begin());
            for (size_t c = 0; c < W; ++c) {
                size_t p = layer * 2 * W + 2 * c;
                double sum = input[c] * double(parameters[p]) + input[(c + s) % W] * double(parameters[p + 1]);
                v[c] = (layer + 1 != depth && sum < 0.0) ? std::expm1(sum) : sum;
            }
        }
    }
    std::vector<float> table(V * W + parameters.size() - config.embedding_parameter_count());
    for (size_t i = 0; i < V * W; ++i) table[i] = float(vec[i]);
    std::copy(parameters.begin() + config.embedding_parameter_count(), parameters.end(),
              table.begin() + V * W);
    validate_finite(table.data(), table.size(), "tabulated parameters");
    return table;
}

uint64_t Random::next_u64() {
    state_ += 0x9e3779b97f4a7c15ULL;
    uint64_t bits = state_;
    bits = (bits ^ (bits >> 30)) * 0xbf58476d1ce4e5b9ULL;
    bits = (bits ^ (bits >> 27)) * 0x94d049bb133111ebULL;
    return bits ^ (bits >> 31);
}

float Random::unit() { return float(uint32_t(next_u64() >> 40)) / 16777216.0f; }

size_t Random::index(size_t bound) {
    uint64_t b = bound;
    uint64_t threshold = (0 - b) % b;
    for (;;) {
        uint64_t bits = next_u64();
        if (bits >= threshold) return size_t(bits % b);
    }
}

void validate_finite(const float *values, size_t n, const char *name) {
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(values[i]))
            throw Error(std::string(name) + " must contain only finite values", kNonfinite);
}

// ---------------------------------------------------------------- text

std::vector<uint32_t> utf8_decode(const std::string &text) {
    std::vector<uint32_t> out;
    const auto *s = reinterpret_cast<const unsigned char *>(text.data());
    size_t n = text.size(), i = 0;
    while (i < n) {
        uint32_t c = s[i];
        size_t extra;
        uint32_t minimum;
        if (c < 0x80) {
            extra = 0;
            minimum = 0;
        } else if ((c & 0xE0) == 0xC0) {
            extra = 1;
            c &= 0x1F;
            minimum = 0x80;
        } else if ((c & 0xF0) == 0xE0) {
            extra = 2;
            c &= 0x0F;
            minimum = 0x800;
        } else if ((c & 0xF8) == 0xF0) {
            extra = 3;
            c &= 0x07;
            minimum = 0x10000;
        } else {
            throw Error("text must be valid UTF-8");
        }
        for (size_t k = 1; k <= extra; ++k) {
            if (i + k >= n || (s[i + k] & 0xC0) != 0x80) throw Error("text must be valid UTF-8");
            c = (c << 6) | (s[i + k] & 0x3F);
        }
        if (c < minimum || c > 0x10FFFF || (c >= 0xD800 && c <= 0xDFFF))
            throw Error("text must be valid UTF-8");
        out.push_back(c);
        i += extra + 1;
    }
    return out;
}

std::string utf8_encode(const uint32_t *scalars, size_t n) {
    std::string out;
    for (size_t i = 0; i < n; ++i) {
        uint32_t c = scalars[i];
        if (c < 0x80) {
            out += char(c);
        } else if (c < 0x800) {
            out += char(0xC0 | (c >> 6));
            out += char(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            out += char(0xE0 | (c >> 12));
            out += char(0x80 | ((c >> 6) & 0x3F));
            out += char(0x80 | (c & 0x3F));
        } else {
            out += char(0xF0 | (c >> 18));
            out += char(0x80 | ((c >> 12) & 0x3F));
            out += char(0x80 | ((c >> 6) & 0x3F));
            out += char(0x80 | (c & 0x3F));
        }
    }
    return out;
}

// Debug rendering of a char as the reference's `{character:?}` prints it.
static std::string debug_char(uint32_t c) {
    switch (c) {
    case '\n': return "'\\n'";
    case '\t': return "'\\t'";
    case '\r': return "'\\r'";
    case '\0': return "'\\0'";
    case '\'': return "'\\''";
    case '\\': return "'\\\\'";
    default: break;
    }
    if (c < 0x20 || (c >= 0x7F && c < 0xA0) || (c >= 0xE000 && c <= 0xF8FF)) {
        char buf[32];
        std::snprintf(buf, sizeof buf, "'\\u{%x}'", c);
        return buf;
    }
    return "'" + utf8_encode(&c, 1) + "'";
}

CharacterTokenizer CharacterTokenizer::from_text(const std::string &utf8) {
    std::vector<uint32_t> scalars = utf8_decode(utf8);
    std::set<uint32_t> unique(scalars.begin(), scalars.end());
    return from_characters(std::vector<uint32_t>(unique.begin(), unique.end()));
}

CharacterTokenizer CharacterTokenizer::from_characters(std::vector<uint32_t> characters) {
    std::set<uint32_t> unique(characters.begin(), characters.end());
    if (characters.size() < 2 || characters.size() > kModelMaxVocab || unique.size() != characters.size())
        throw Error("tokenizer must contain 2..65536 unique characters");
    for (uint32_t c : characters)
        if (c > 0x10FFFF || (c >= 0xD800 && c <= 0xDFFF)) throw Error("invalid checkpoint character");
    CharacterTokenizer t;
    t.characters_ = std::move(characters);
    return t;
}

std::vector<uint32_t> CharacterTokenizer::encode(const std::string &utf8) const {
    std::vector<uint32_t> out;
    for (uint32_t c : utf8_decode(utf8)) {
        auto it = std::find(characters_.begin(), characters_.end(), c);
        if (it == characters_.end())
            throw Error("character " + debug_char(c) + " is outside the tokenizer vocabulary");
        out.push_back(uint32_t(it - characters_.begin()));
    }
    return out;
}

std::string CharacterTokenizer::decode(const uint32_t *tokens, size_t n) const {
    std::vector<uint32_t> scalars(n);
    for (size_t i = 0; i < n; ++i) {
        if (tokens[i] >= characters_.size()) throw Error("token ID is outside the tokenizer vocabulary");
        scalars[i] = characters_[tokens[i]];
    }
    return utf8_encode(scalars.data(), n);
}

// ---------------------------------------------------------- checkpoint

static void put_u32(std::vector<uint8_t> &out, uint32_t v) {
    for (int i = 0; i < 4; ++i) out.push_back(uint8_t(v >> (8 * i)));
}

std::vector<uint8_t> Checkpoint::serialize() const {
    if (config.long_context)
        throw Error("long-context configurations cannot be stored in a checkpoint");
    if (config.parameter_count() != parameters.size() || config.vocab_size != tokenizer.vocab_size())
        throw Error("checkpoint model, parameters, and tokenizer do not match");
    validate_finite(parameters.data(), parameters.size(), "checkpoint parameters");
    Layout::build(config).validate_constraints(config, parameters.data());
    bool table = config.embedding == TokenEmbedding::Table;
    bool butterfly = config.connectivity == MeshConnectivity::Butterfly;
    bool v09 = !config.reference_operators();
    bool is_default = !table && !butterfly && !v09;
    std::vector<uint8_t> out;
    const char *magic = v09 ? "MSHGPT09" : (is_default ? "MSHGPT07" : "MSHGPT08");
    out.insert(out.end(), magic, magic + 8);
    for (size_t field : {config.vocab_size, config.context, config.width, config.heads, config.layers,
                         config.attention_mesh_depth, config.ffn_mesh_depth})
        put_u32(out, uint32_t(field));
    if (!is_default) {
        put_u32(out, table ? 1 : 0);
        put_u32(out, butterfly ? 1 : 0);
    }
    if (v09) {
        // Field order of checkpoint.rs:61-78.
        const EmbeddingGeometry &g = config.geometry;
        uint32_t overlap;
        std::memcpy(&overlap, &g.overlap, 4);
        for (uint32_t field : {uint32_t(g.form), uint32_t(g.order), uint32_t(g.frequency), uint32_t(g.harmonics),
                               overlap, uint32_t(g.normalization), uint32_t(g.frozen), uint32_t(g.preserve_features),
                               uint32_t(g.modulus), uint32_t(g.seed), uint32_t(g.seed >> 32), uint32_t(config.rope),
                               uint32_t(config.qk_norm), uint32_t(config.xsa)})
            put_u32(out, field);
    }
    for (uint32_t c : tokenizer.characters()) put_u32(out, c);
    for (float p : parameters) {
        uint32_t bits;
        std::memcpy(&bits, &p, 4);
        put_u32(out, bits);
    }
    return out;
}

void Checkpoint::save(const std::string &path) const {
    std::vector<uint8_t> bytes = serialize();
    std::ofstream file(path, std::ios::binary | std::ios::trunc);
    if (!file) throw Error("cannot create checkpoint " + path, kIo);
    file.write(reinterpret_cast<const char *>(bytes.data()), std::streamsize(bytes.size()));
    if (!file) throw Error("cannot write checkpoint " + path, kIo);
}

namespace {
struct Reader {
    const uint8_t *p;
    size_t n, at = 0;
    uint32_t word() {
        if (n - at < 4) throw Error("failed to fill whole buffer", kIo);
        uint32_t v = uint32_t(p[at]) | uint32_t(p[at + 1]) << 8 | uint32_t(p[at + 2]) << 16 |
                     uint32_t(p[at + 3]) << 24;
        at += 4;
        return v;
    }
};

bool read_switch(uint32_t code) {
    if (code > 1) throw Error("invalid checkpoint switch");
    return code == 1;
}
}  // namespace

Checkpoint Checkpoint::read(const uint8_t *bytes, size_t n) {
    if (n < 8) throw Error("failed to fill whole buffer", kIo);
    std::string magic(reinterpret_cast<const char *>(bytes), 8);
    bool v07 = magic == "MSHGPT07", v08 = magic == "MSHGPT08", v09 = magic == "MSHGPT09";
    if (!v07 && !v08 && !v09) {
        if (magic == "MSHGPT01" || magic == "MSHGPT02")
            throw Error("checkpoint uses learned position embeddings; retrain Mesh GPT with RoPE");
        if (magic == "MSHGPT03") throw Error("checkpoint uses LayerNorm; retrain Mesh GPT with RMSNorm");
        if (magic == "MSHGPT04") throw Error("checkpoint contains biases; retrain bias-free Mesh GPT");
        if (magic == "MSHGPT05")
            throw Error("checkpoint uses learned RMSNorm without QK-Norm; retrain Mesh GPT with "
                        "parameter-free QK-Norm");
        if (magic == "MSHGPT06")
            throw Error("checkpoint uses a learned token table; retrain Mesh GPT with mesh token "
                        "embeddings");
        throw Error("unsupported Mesh GPT checkpoint format");
    }
    Reader r{bytes, n, 8};
    Checkpoint ck;
    GptConfig &c = ck.config;
    c.vocab_size = r.word();
    c.context = r.word();
    c.width = r.word();
    c.heads = r.word();
    c.layers = r.word();
    c.attention_mesh_depth = r.word();
    c.ffn_mesh_depth = r.word();
    if (v08 || v09) {
        uint32_t e = r.word();
        if (e > 1) throw Error("unknown checkpoint token embedding");
        c.embedding = TokenEmbedding(e);
        uint32_t k = r.word();
        if (k > 1) throw Error("unknown checkpoint mesh connectivity");
        c.connectivity = MeshConnectivity(k);
        if (v08 && c.embedding == TokenEmbedding::Mesh && c.connectivity == MeshConnectivity::Neighbor)
            throw Error("the default architecture must use the MSHGPT07 layout");
    }
    if (v09) {
        // Field order and code ranges of checkpoint.rs:146-168, geometry.rs:37-47.
        uint32_t form = r.word();
        if (form > 9) throw Error("unknown checkpoint EmbeddingForm: " + std::to_string(form));
        uint32_t order = r.word();
        if (order > 2) throw Error("unknown checkpoint EmbeddingOrder: " + std::to_string(order));
        uint32_t frequency = r.word(), harmonics = r.word(), overlap = r.word();
        uint32_t norm = r.word();
        if (norm > 2) throw Error("unknown checkpoint EmbeddingNorm: " + std::to_string(norm));
        bool frozen = read_switch(r.word());
        uint32_t preserve = r.word(), modulus = r.word(), seed_lo = r.word(), seed_hi = r.word();
        EmbeddingGeometry &g = c.geometry;
        g.form = EmbeddingForm(form);
        g.order = EmbeddingOrder(order);
        g.frequency = frequency;
        g.harmonics = harmonics;
        std::memcpy(&g.overlap, &overlap, 4);
        g.normalization = EmbeddingNorm(norm);
        g.frozen = frozen;
        g.preserve_features = preserve;
        g.modulus = modulus;
        g.seed = uint64_t(seed_lo) | uint64_t(seed_hi) << 32;
        c.rope = read_switch(r.word());
        c.qk_norm = read_switch(r.word());
        c.xsa = read_switch(r.word());
        if (g.is_default() && c.rope && c.qk_norm && c.xsa)
            throw Error("default geometry must use an older checkpoint layout");
    }
    size_t count = c.parameter_count();
    std::vector<uint32_t> characters(c.vocab_size);
    for (auto &ch : characters) {
        ch = r.word();
        if (ch > 0x10FFFF || (ch >= 0xD800 && ch <= 0xDFFF)) throw Error("invalid checkpoint character");
    }
    ck.tokenizer = CharacterTokenizer::from_characters(characters);
    ck.parameters.resize(count);
    for (auto &p : ck.parameters) {
        uint32_t bits = r.word();
        std::memcpy(&p, &bits, 4);
    }
    validate_finite(ck.parameters.data(), count, "checkpoint parameters");
    Layout::build(c).validate_constraints(c, ck.parameters.data());
    if (r.at != n) throw Error("unexpected trailing checkpoint bytes");
    return ck;
}

Checkpoint Checkpoint::load(const std::string &path) {
    std::ifstream file(path, std::ios::binary);
    if (!file) throw Error("cannot open checkpoint " + path + ": No such file or directory", kIo);
    std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(file)), std::istreambuf_iterator<char>());
    return read(bytes.data(), bytes.size());
}

}  // namespace meshgpt
